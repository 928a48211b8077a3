"""ctypes binding of libhq.so (include/hq.h).

The library is the only compute path: there is no host fallback.  Loading
fails with an error when libhq.so is missing, and every call checks the
returned status.  Reference binding this replaces: cpu_lightspark.py:45-111
(reference repository), which loads its native library with ctypes.CDLL and
declares argtypes the same way.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libhq.so"

vp = ctypes.c_void_p
c_int = ctypes.c_int
c_float = ctypes.c_float
c_size = ctypes.c_size_t


class HqLayer(ctypes.Structure):
    _fields_ = [(name, vp) for name in (
        "qkv", "qkv_scales", "o", "o_scales", "gate_up", "gate_up_scales",
        "down", "down_scales", "input_norm", "post_norm", "q_norm", "k_norm")]


class HqModel(ctypes.Structure):
    _fields_ = [
        ("layers", ctypes.c_int32), ("hidden", ctypes.c_int32),
        ("intermediate", ctypes.c_int32), ("heads", ctypes.c_int32),
        ("kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("vocab", ctypes.c_int32), ("rope_positions", ctypes.c_int32),
        ("eps", ctypes.c_float), ("flags", ctypes.c_int32),
        ("layer", ctypes.POINTER(HqLayer)),
        ("embedding", vp), ("embedding_scales", vp), ("final_norm", vp),
        ("rope_cos", vp), ("rope_sin", vp),
        ("device_layer", vp),
    ]


class HqState(ctypes.Structure):
    _fields_ = [
        ("capacity", ctypes.c_int32), ("reserved", ctypes.c_int32),
        ("keys", vp), ("values", vp), ("position", vp), ("token", vp), ("status", vp),
        ("x", vp), ("qkv", vp), ("attended", vp), ("activated", vp), ("logits", vp),
        ("workspace", vp),
    ]


HQ_STEP_BAD_TOKEN = 1
HQ_STEP_FULL = 2
HQ_STEP_SYNC = 4
HQ_MODEL_PER_LAYER_KERNELS = 1

_SIGNATURES = {
    "hq_status_string": ([c_int], ctypes.c_char_p),
    "hq_abi_version": ([], c_int),
    "hq_int4_i8_gemv": ([vp, vp, vp, c_float, vp, c_int, c_int, vp], c_int),
    "hq_quant_int4_gemv": ([vp, vp, vp, vp, c_int, c_int, vp, vp, vp, vp], c_int),
    "hq_quantize_activation": ([vp, c_int, vp, vp, vp], c_int),
    "hq_rmsnorm": ([vp, vp, vp, c_int, c_float, vp], c_int),
    "hq_gqa_workspace_bytes": ([c_int, c_int, c_int, c_int], c_size),
    "hq_gqa_decode": ([vp, vp, vp, vp, vp, c_int, c_int, c_int, c_int, c_int, vp], c_int),
    "hq_gqa_decode_noalloc": ([vp, vp, vp, vp, c_int, c_int, c_int, c_int, c_int, vp], c_int),
    "hq_argmax_workspace_bytes": ([c_int], c_size),
    "hq_argmax": ([vp, c_int, vp, vp, vp], c_int),
    "hq_sample_workspace_bytes": ([c_int, c_int], c_size),
    "hq_sample_token": ([vp, c_int, vp, c_int, c_float, c_float, c_int, c_float, vp, vp, vp, vp, vp, vp], c_int),
    "hq_gemm_workspace_bytes": ([c_int, c_int, c_int], c_size),
    "hq_int4_i8_gemm": ([vp, vp, vp, vp, vp, c_int, c_int, c_int, vp, vp, vp], c_int),
    "hq_quant_int4_gemm": ([vp, vp, vp, vp, c_int, c_int, c_int, vp, vp, vp, vp, vp], c_int),
    "hq_step_layer_blocks": ([ctypes.POINTER(HqModel)], c_int),
    "hq_step_workspace_bytes": ([ctypes.POINTER(HqModel), c_int], c_size),
    "hq_decode_step": ([ctypes.POINTER(HqModel), ctypes.POINTER(HqState), vp], c_int),
    "hq_prefill_workspace_bytes": ([ctypes.POINTER(HqModel), c_int], c_size),
    "hq_prefill": ([ctypes.POINTER(HqModel), ctypes.POINTER(HqState), vp, c_int, c_int, vp, vp], c_int),
    "hq_decode_batch_workspace_bytes": ([ctypes.POINTER(HqModel), c_int], c_size),
    "hq_decode_batch": ([ctypes.POINTER(HqModel), ctypes.POINTER(HqState), c_int, c_int, vp, vp], c_int),
    "hq_step_gemv": ([ctypes.POINTER(HqModel), ctypes.POINTER(HqState), c_int, c_int, vp], c_int),
    "hq_step_layers": ([ctypes.POINTER(HqModel), ctypes.POINTER(HqState), vp], c_int),
    "hq_graph_capture": ([ctypes.POINTER(HqModel), ctypes.POINTER(HqState), c_int, vp,
                          ctypes.POINTER(vp)], c_int),
    "hq_graph_launch": ([vp, vp], c_int),
    "hq_graph_destroy": ([vp], c_int),
}

_LIB = None


def lib() -> ctypes.CDLL:
    """Load libhq.so; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m harsh4b_amd.build` "
                "(the HIP kernels are the only compute path; there is no fallback)")
        library = ctypes.CDLL(str(LIB_PATH))
        for name, (argtypes, restype) in _SIGNATURES.items():
            fn = getattr(library, name)
            fn.argtypes = argtypes
            fn.restype = restype
        _LIB = library
    return _LIB


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def check(status: int, what: str) -> None:
    if status != 0:
        text = lib().hq_status_string(status).decode()
        raise RuntimeError(f"{what} failed: {text} (status {status})")
