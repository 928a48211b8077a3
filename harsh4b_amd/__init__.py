"""harsh4b_amd - MI355X (gfx950) int4 decode hot path of OneBit-AI/Harsh4B.

libhq.so (HIP kernels + C ABI, include/hq.h) does all arithmetic; the Python
side mirrors the reference's cpu_lightspark.py call surface.
"""
__all__ = ["lightspark", "synthetic", "config", "build"]
