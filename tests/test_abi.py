"""CPU-side checks of the product boundary: libhq.so loads and exports every
symbol include/hq.h declares, and the host mirror keeps the reference's
layout and error behaviour (cpu_lightspark.py in the reference repository).
No GPU calls are made here."""
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    text = (ROOT / "include" / "hq.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hq_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from harsh4b_amd import _native
    lib = _native.lib()
    names = declared_symbols()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(_native.exported_symbols())


def test_status_strings_and_version():
    from harsh4b_amd import _native
    lib = _native.lib()
    assert lib.hq_abi_version() == 101
    assert lib.hq_status_string(0) == b"ok"
    assert b"invalid" in lib.hq_status_string(1)


def test_host_validation_rejects_bad_shapes_without_launching():
    import ctypes
    # These return before any HIP call, so they run without a GPU.
    from harsh4b_amd import _native
    lib = _native.lib()
    assert lib.hq_int4_i8_gemv(None, None, None, 1.0, None, 4, 3, None) == 1      # odd width
    assert lib.hq_quant_int4_gemv(None, None, None, None, 4, 0, None, None, None, None) == 1
    assert lib.hq_int4_i8_gemv(None, None, None, 1.0, None, 0, 64, None) == 0    # empty: no-op
    assert lib.hq_gqa_decode(None, None, None, None, None, 1, 1, 1, 16, 16, None) == 1
    # score_stride (the reference's scores row stride, state.capacity) below
    # the context is refused before any launch
    buf = ctypes.create_string_buffer(1024)
    p = ctypes.addressof(buf)
    ws = (p + 255) & ~255
    assert lib.hq_gqa_decode(p, p, p, ws, p, 10, 8, 4, 128, 9, None) == 1
    assert lib.hq_gqa_decode(p, p, p, ws + 16, p, 10, 8, 4, 128, 10, None) == 2
    # the workspace is sized by score_stride, like the reference's scores
    # 32 heads x 64 chunks x (128 o + m, l + the second combine unit's m, l copies)
    assert lib.hq_gqa_workspace_bytes(4096, 8, 4, 128) == 256 + 32 * 64 * 132 * 4
    # the no-allocation variant: same checks, and contexts whose chunk
    # partials exceed its 4 MiB device array are refused before any HIP call
    assert lib.hq_gqa_decode_noalloc(p, p, p, p, 10, 8, 4, 128, 9, None) == 1
    assert lib.hq_gqa_decode_noalloc(None, p, p, p, 10, 8, 4, 128, 10, None) == 1
    assert lib.hq_gqa_decode_noalloc(p, p, p, p, 15873, 8, 4, 128, 20000, None) == 1
    assert lib.hq_gemm_workspace_bytes(0, 1, 1) == 0
    assert lib.hq_gqa_workspace_bytes(64, 8, 4, 128) >= 32 * 132 * 4


def test_sampler_rejects_bad_arguments_without_launching():
    # every check returns before a HIP call; the pointers are never read
    import ctypes
    from harsh4b_amd import _native
    lib = _native.lib()
    buf = ctypes.create_string_buffer(1024)
    p = ctypes.addressof(buf)
    ws = (p + 255) & ~255

    def call(n=1000, top_k=40, temperature=0.7, rp=1.08, top_p=0.9, workspace=ws, n_generated=0):
        return lib.hq_sample_token(p, n, p, n_generated, rp, temperature, top_k, top_p, p, p, None, None,
                                   workspace, None)

    assert call(top_k=0) == 1 and call(top_k=2049) == 1
    assert call(temperature=0.0) == 1 and call(temperature=float("nan")) == 1
    assert call(rp=0.0) == 1 and call(top_p=0.0) == 1 and call(top_p=-1.0) == 1
    assert call(n=0) == 1 and call(n_generated=-1) == 1
    assert call(workspace=ws + 4) == 2                                          # 256-byte alignment
    assert lib.hq_sample_token(None, 10, None, 0, 1.0, 1.0, 5, 1.0, p, p, None, None, ws, None) == 1
    # the ticket counter, then k candidate keys per 4096-logit slice
    assert lib.hq_sample_workspace_bytes(151936, 40) >= 4 + 38 * 40 * 8
    assert lib.hq_sample_workspace_bytes(10, 40) >= 4 + 10 * 8


def test_sampler_host_checks():
    torch = pytest.importorskip("torch")
    from harsh4b_amd import lightspark as ls

    class Args:
        argmax, repetition_penalty, temperature, top_k, top_p = False, 1.08, 0.7, 40, 0.9
    with pytest.raises(ValueError, match="Generator"):
        ls.sample_logits(torch.zeros(4), [], Args())
    with pytest.raises(ValueError, match="device tensor"):
        ls.sample_token(torch.zeros(4), [], 1.0, 1.0, 2, 1.0, 0.5)


def test_workspace_sizes_cover_qwen_step():
    import ctypes
    from harsh4b_amd import _native
    from harsh4b_amd.config import QWEN3_4B
    m = _native.HqModel()
    m.layers, m.hidden, m.intermediate = 36, 2560, 9728
    m.heads, m.kv_heads, m.head_dim, m.vocab = 32, 8, 128, 151936
    nbytes = _native.lib().hq_step_workspace_bytes(ctypes.byref(m), 4160)
    # attention partials 32 heads x 65 chunks x 130 floats + LM head partials
    # (one value and one index per block of the persistent 512-block launch)
    assert nbytes >= 32 * 65 * 130 * 4 + 2 * 512 * 4


def test_pack_int4_mirror_matches_reference_layout(kat):
    from harsh4b_amd.lightspark import pack_int4
    np.testing.assert_array_equal(pack_int4(kat["pack_w"]), kat["pack_p"])
    with pytest.raises(ValueError, match=r"\[-7,\+7\]"):
        pack_int4(np.array([[8, 0]], dtype=np.int8))
    with pytest.raises(ValueError, match="even width"):
        pack_int4(np.zeros((1, 3), dtype=np.int8))


def test_rope_tables_mirror(forward_golden):
    from harsh4b_amd.lightspark import rope_tables
    cos, sin = rope_tables(forward_golden["config"])
    np.testing.assert_array_equal(cos, forward_golden["rope_cos"])
    np.testing.assert_array_equal(sin, forward_golden["rope_sin"])


def test_qwen_body_bytes():
    from harsh4b_amd.config import QWEN3_4B, body_bytes, shapes
    assert body_bytes(QWEN3_4B) == 1_816_657_920
    assert shapes(QWEN3_4B)["qkv"] == (6144, 2560)
    assert shapes(QWEN3_4B)["gate_up"] == (19456, 2560)


def test_product_package_never_imports_the_oracle():
    pkg = ROOT / "harsh4b_amd"
    for path in list(pkg.rglob("*.py")) + list(pkg.rglob("*.hip")) + list(pkg.rglob("*.h")):
        text = path.read_text()
        assert "import oracle" not in text and "from oracle" not in text, path
        assert "liborhq" not in text, path
