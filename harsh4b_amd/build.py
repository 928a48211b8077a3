"""Build libhq.so (the HIP kernels + C ABI) in-tree for gfx950.

Each ``csrc/*.hip`` translation unit is compiled with hipcc in parallel and
linked into ``harsh4b_amd/lib/libhq.so``.  Flags that matter for results:
  -ffp-contract=off                 no implicit FMA: the fp32 spec is written
                                    with explicit fmaf where it wants one;
  -target-feature -packed-fp32-ops  no v_pk_*_f32 generated from scalar code.
Run: python -m harsh4b_amd.build            (libhq.so)
     python -m harsh4b_amd.build --trace    (also libhq_trace.so: the same
     sources with HQ_ENGINE_TRACE, whose layer kernel records per-phase
     timestamps for harsh4b_amd.profile)
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
LIB = LIBDIR / "libhq.so"
TRACE_LIB = LIBDIR / "libhq_trace.so"
ARCH = os.environ.get("HQ_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Wall", "-Wno-unused-parameter",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: the HIP toolchain is required to build libhq.so")
    return exe


def _compile(src: Path, obj: Path, defines=()) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *defines, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = True, trace: bool = False) -> Path:
    """Compile every csrc/*.hip and link libhq.so (always rebuilds); with
    trace, libhq_trace.so from the same sources with HQ_ENGINE_TRACE."""
    sources = sorted(CSRC.glob("*.hip"))
    objdir = PKG / ("_build_trace" if trace else "_build")
    lib = TRACE_LIB if trace else LIB
    defines = ("-DHQ_ENGINE_TRACE",) if trace else ()
    objdir.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    objs = [objdir / (s.stem + ".o") for s in sources]
    workers = min(len(sources), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        list(ex.map(lambda so: _compile(*so, defines), zip(sources, objs)))
    tmp = lib.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib} from {len(sources)} HIP sources")
    return lib


if __name__ == "__main__":
    build()
    if "--trace" in sys.argv[1:]:
        build(trace=True)
