"""CPU oracle pins: golden vectors of the reference's tests, closed forms in
float64, numpy's own IEEE conversions, and brute force on small inputs.

The reference tests cited are tests/test_cpu_lightspark.py in the reference
repository; the kernels are cpu_kernels/litespark_int4.cpp.
"""
import math

import numpy as np
import pytest

import oracle


# ----------------------------------------------------------------- packing
def test_pack_golden_and_range_error(kat):
    np.testing.assert_array_equal(oracle.pack_int4(kat["pack_w"]), kat["pack_p"])
    with pytest.raises(ValueError, match=r"\[-7,\+7\]"):
        oracle.pack_int4(np.array([[8, 0]], dtype=np.int8))
    with pytest.raises(ValueError, match=r"\[-7,\+7\]"):
        oracle.pack_int4(np.array([[0, -8]], dtype=np.int8))
    with pytest.raises(ValueError, match="even width"):
        oracle.pack_int4(np.zeros((2, 3), dtype=np.int8))


def test_pack_unpack_roundtrip_and_nibble_layout():
    rng = np.random.default_rng(5)
    w = rng.integers(-7, 8, size=(13, 46), dtype=np.int8)
    p = oracle.pack_int4(w)
    np.testing.assert_array_equal(oracle.unpack_int4(p, 46), w)
    # low nibble = even column, high nibble = odd column, two's complement
    lo = (p & 0xF).astype(np.int16)
    hi = (p >> 4).astype(np.int16)
    np.testing.assert_array_equal(np.where(lo > 7, lo - 16, lo), w[:, 0::2])
    np.testing.assert_array_equal(np.where(hi > 7, hi - 16, hi), w[:, 1::2])


# ----------------------------------------------------------------- GEMV
def test_gemv_known_answer(kat):
    w = kat["gemv_w"]
    p = oracle.pack_int4(w)
    out = oracle.int4_i8_gemv(kat["gemv_x"], p, kat["gemv_scales"], float(kat["gemv_act"]),
                              w.shape[0], w.shape[1])
    np.testing.assert_allclose(out, kat["gemv_expected"], rtol=2e-6, atol=2e-5)
    acc = oracle.int4_i8_gemv_acc(kat["gemv_x"], p, w.shape[0], w.shape[1])
    np.testing.assert_array_equal(acc, kat["gemv_acc"])


@pytest.mark.parametrize("rows,width", [(1, 2), (3, 30), (63, 64), (64, 64), (67, 200),
                                        (130, 2562), (9, 4096)])
def test_gemv_brute_force(rows, width):
    rng = np.random.default_rng(rows * 1000 + width)
    w = rng.integers(-7, 8, size=(rows, width), dtype=np.int8)
    x = rng.integers(-127, 128, size=width, dtype=np.int8)
    acc = oracle.int4_i8_gemv_acc(x, oracle.pack_int4(w), rows, width)
    np.testing.assert_array_equal(acc, w.astype(np.int64) @ x.astype(np.int64))


def test_gemv_extremes_do_not_overflow():
    width = 9728
    w = np.full((2, width), 7, dtype=np.int8)
    w[1] = -7
    x = np.full(width, 127, dtype=np.int8)
    acc = oracle.int4_i8_gemv_acc(x, oracle.pack_int4(w), 2, width)
    assert acc.tolist() == [7 * 127 * width, -7 * 127 * width]


def test_gemv_epilogue_order():
    # litespark_int4.cpp:73-74: ((float)acc * act) * scale, two roundings.
    rng = np.random.default_rng(8)
    w = rng.integers(-7, 8, size=(300, 64), dtype=np.int8)
    x = rng.integers(-127, 128, size=64, dtype=np.int8)
    s = rng.random(300, dtype=np.float32)
    act = np.float32(0.0123)
    out = oracle.int4_i8_gemv(x, oracle.pack_int4(w), s, act, 300, 64)
    acc = (w.astype(np.int64) @ x.astype(np.int64)).astype(np.float32)
    np.testing.assert_array_equal(out, (acc * act) * s)


def test_batched_gemm_equals_independent_gemvs():
    rng = np.random.default_rng(9)
    w = rng.integers(-7, 8, size=(40, 96), dtype=np.int8)
    x = rng.integers(-127, 128, size=(8, 96), dtype=np.int8)
    acc = oracle.int4_i8_gemm_acc(x, oracle.pack_int4(w), 40, 96)
    np.testing.assert_array_equal(acc, x.astype(np.int64) @ w.astype(np.int64).T)


# ----------------------------------------------------------------- quantization
def test_quantize_closed_form():
    rng = np.random.default_rng(11)
    x = rng.standard_normal(2560).astype(np.float32)
    q, s = oracle.quantize_activation(x)
    amax = np.float32(np.abs(x).max())
    inv = np.float32(127.0) / amax
    expected = np.clip(np.rint(x * inv), -127, 127).astype(np.int8)
    np.testing.assert_array_equal(q, expected)
    assert s == amax / np.float32(127.0)
    i = int(np.abs(x).argmax())
    assert abs(int(q[i])) == 127
    # dequantization error bounded by half a step
    assert np.max(np.abs(q.astype(np.float64) * float(s) - x)) <= 0.5 * float(s) * (1 + 1e-5)


def test_quantize_zero_and_tiny_vectors():
    q, s = oracle.quantize_activation(np.zeros(64, dtype=np.float32))
    assert not q.any() and s == np.float32(1e-5) / np.float32(127)
    x = np.full(8, 1e-7, dtype=np.float32)
    q, s = oracle.quantize_activation(x)
    assert s == np.float32(1e-5) / np.float32(127)
    np.testing.assert_array_equal(q, np.rint(x * (np.float32(127) / np.float32(1e-5))).astype(np.int8))


def test_quantize_ties_round_half_even():
    x = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5], dtype=np.float32)
    q, _ = oracle.quantize_activation(x)   # amax 127 -> inv 1
    assert q.tolist() == [127, 0, 2, 2, 0, -2]


# ----------------------------------------------------------------- norms
def test_rmsnorm_against_float64():
    rng = np.random.default_rng(12)
    x = (rng.standard_normal(2560) * 3).astype(np.float32)
    g = rng.uniform(0.5, 1.5, 2560).astype(np.float32)
    y = oracle.rmsnorm(x, g, 1e-6)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 * x64) + 1e-6) * g
    np.testing.assert_allclose(y, ref, rtol=2e-6, atol=1e-7)


def test_rmsnorm_tree_is_not_sequential_sum():
    # A plausible slip (summing sequentially) changes bits on large inputs;
    # the 256-lane tree must match its definition exactly.
    rng = np.random.default_rng(13)
    x = (rng.standard_normal(2560) * 10).astype(np.float32)
    g = np.ones(2560, dtype=np.float32)
    lanes = np.zeros(256, dtype=np.float32)
    for l in range(256):
        p = np.float32(0)
        for v in x[l::256]:
            p = np.float32(np.float64(v) * np.float64(v) + np.float64(p))  # exact fma in f64
        lanes[l] = p
    o = 128
    while o >= 1:
        lanes[:o] = lanes[:o] + lanes[o:2 * o]
        o //= 2
    r = np.sqrt(lanes[0] / np.float32(2560) + np.float32(1e-6))
    np.testing.assert_array_equal(oracle.rmsnorm(x, g, 1e-6), (x / r) * g)


def test_head_norm_and_rope_against_float64():
    rng = np.random.default_rng(14)
    x = rng.standard_normal((8, 128)).astype(np.float32) * 2
    g = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    y = oracle.head_norm(x, g, 1e-6)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 * x64, axis=1, keepdims=True) + 1e-6) * g
    np.testing.assert_allclose(y, ref, rtol=2e-6, atol=1e-7)
    ang = rng.uniform(-3, 3, 64)
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    r = oracle.rope(y, c, s)
    y64 = y.astype(np.float64)
    ref1 = y64[:, :64] * c - y64[:, 64:] * s
    ref2 = y64[:, 64:] * c + y64[:, :64] * s
    np.testing.assert_allclose(r, np.concatenate([ref1, ref2], axis=1), rtol=1e-6, atol=1e-6)
    # a rotation keeps each pair's norm
    n0 = y64[:, :64] ** 2 + y64[:, 64:] ** 2
    n1 = r[:, :64].astype(np.float64) ** 2 + r[:, 64:].astype(np.float64) ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-5)


# ----------------------------------------------------------------- spec exp / fp16
def _ulp_err(a32, ref64):
    a = a32.astype(np.float64)
    ulp = np.spacing(np.abs(ref64).astype(np.float32)).astype(np.float64)
    return np.abs(a - ref64) / ulp


def test_expf_accuracy_and_specials():
    rng = np.random.default_rng(15)
    x = np.concatenate([rng.uniform(-87, 88.7, 20000), rng.uniform(-1, 1, 5000),
                        np.array([0.0, -0.0, 1.0, -1.0, 88.72, -86.99])]).astype(np.float32)
    y = oracle.expf(x)
    err = _ulp_err(y, np.exp(x.astype(np.float64)))
    assert err.max() <= 1.0, err.max()
    assert oracle.expf(np.float32([0.0]))[0] == 1.0
    sp = oracle.expf(np.array([np.inf, -np.inf, 100.0, -100.0, -87.5], dtype=np.float32))
    assert sp[0] == np.inf and sp[1] == 0 and sp[2] == np.inf and sp[3] == 0 and sp[4] == 0
    assert np.isnan(oracle.expf(np.array([np.nan], dtype=np.float32))[0])


def test_cody_waite_split_is_ln2():
    hi, lo = float.fromhex("0x1.62e400p-1"), float.fromhex("0x1.7f7d1cp-20")
    assert abs(hi + lo - math.log(2)) < 1e-13
    assert (np.float32(hi).view(np.uint32) & 0xFF) == 0   # hi*n exact for |n| < 2^8


def test_f16_conversion_matches_numpy():
    rng = np.random.default_rng(16)
    x = np.concatenate([
        rng.standard_normal(50000).astype(np.float32),
        (rng.standard_normal(20000) * 1e-5).astype(np.float32),     # subnormal halves
        (rng.standard_normal(5000) * 3e4).astype(np.float32),       # near overflow
        np.array([65504, 65519.99, 65520, 1e-8, 2.0 ** -25, 2.0 ** -24 * 1.5,
                  2.0 ** -24 * 2.5, -0.0, np.inf, -np.inf], dtype=np.float32),
    ])
    bits = oracle.f32_to_f16_bits(x)
    np.testing.assert_array_equal(bits, x.astype(np.float16).view(np.uint16))
    back = oracle.f16_bits_to_f32(bits)
    np.testing.assert_array_equal(back, x.astype(np.float16).astype(np.float32))


# ----------------------------------------------------------------- attention
def test_gqa_known_answer(kat):
    kv, g, ctx, cap, d = (int(v) for v in kat["gqa_shape"])
    out, _ = oracle.gqa_decode_ref(kat["gqa_query"], kat["gqa_keys"], kat["gqa_values"],
                                   ctx, kv, g, d, cap)
    np.testing.assert_allclose(out, kat["gqa_expected"], rtol=2e-5, atol=2e-5)
    split = oracle.gqa_decode_split_f32(kat["gqa_query"], kat["gqa_keys"], kat["gqa_values"],
                                        ctx, kv, g, d)
    np.testing.assert_allclose(split, kat["gqa_expected"], rtol=2e-5, atol=2e-5)


def _attention64(q, k, v, ctx, kv, g, d):
    q64 = q.astype(np.float64).reshape(kv, g, d)
    k64 = k[:ctx].astype(np.float64)
    v64 = v[:ctx].astype(np.float64)
    s = np.einsum("hgd,thd->hgt", q64, k64) / math.sqrt(d)
    s -= s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("hgt,thd->hgd", p, v64).reshape(kv * g, d)


@pytest.mark.parametrize("ctx,chunk", [(1, 64), (63, 64), (64, 64), (65, 64), (300, 64),
                                       (300, 16), (1000, 128)])
def test_gqa_split_against_float64(ctx, chunk):
    rng = np.random.default_rng(ctx + chunk)
    kv, g, d = 8, 4, 128
    q = rng.standard_normal((kv * g, d)).astype(np.float32)
    k = rng.standard_normal((ctx, kv, d)).astype(np.float32)
    v = rng.standard_normal((ctx, kv, d)).astype(np.float32)
    k16, v16 = oracle.f32_to_f16_bits(k), oracle.f32_to_f16_bits(v)
    out = oracle.gqa_decode_split(q, k16, v16, ctx, kv, g, d, chunk)
    ref = _attention64(q, oracle.f16_bits_to_f32(k16), oracle.f16_bits_to_f32(v16), ctx, kv, g, d)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=2e-6)
    ref_alg, _ = oracle.gqa_decode_ref(q, oracle.f16_bits_to_f32(k16), oracle.f16_bits_to_f32(v16),
                                       ctx, kv, g, d, ctx)
    np.testing.assert_allclose(out, ref_alg, rtol=1e-5, atol=2e-6)


def test_gqa_head_mapping():
    # query head h reads kv head h // groups (litespark_int4.cpp:178)
    rng = np.random.default_rng(21)
    kv, g, d, ctx = 2, 3, 16, 5
    q = rng.standard_normal((kv * g, d)).astype(np.float32)
    k = rng.standard_normal((ctx, kv, d)).astype(np.float32)
    v = np.zeros((ctx, kv, d), dtype=np.float32)
    v[:, 1, :] = 1.0    # kv head 1 has all-ones values
    out = oracle.gqa_decode_split_f32(q, k, v, ctx, kv, g, d, 64)
    np.testing.assert_array_equal(out[:3], 0.0)
    np.testing.assert_allclose(out[3:], 1.0, rtol=1e-6)


# ----------------------------------------------------------------- SwiGLU, argmax
def test_swiglu_against_float64():
    rng = np.random.default_rng(22)
    gt = (rng.standard_normal(9728) * 4).astype(np.float32)
    up = (rng.standard_normal(9728) * 4).astype(np.float32)
    gt[:4] = [-100.0, 100.0, 0.0, -0.0]
    out = oracle.swiglu(gt, up)
    g64 = gt.astype(np.float64)
    ref = g64 / (1 + np.exp(-g64)) * up
    np.testing.assert_allclose(out, ref, rtol=3e-7 * 4, atol=1e-30)


def test_argmax_golden_ties_and_nan(kat):
    assert oracle.argmax(kat["argmax_logits"]) == int(kat["argmax_expected"])
    x = np.array([1.0, 5.0, 5.0, 2.0], dtype=np.float32)
    assert oracle.argmax(x) == int(np.argmax(x)) == 1
    y = np.array([1.0, np.nan, 9.0, np.nan], dtype=np.float32)
    assert oracle.argmax(y) == int(np.argmax(y)) == 1
    z = np.array([-0.0, 0.0], dtype=np.float32)
    assert oracle.argmax(z) == int(np.argmax(z)) == 0


# ----------------------------------------------------------------- GEMV vector path
@pytest.mark.parametrize("rows,width", [(1, 2), (3, 126), (5, 128), (7, 130), (64, 2560), (33, 4162),
                                        (17, 9728)])
def test_gemv_vector_path_equals_scalar(rows, width):
    """The AVX-512 VNNI path (used where the CPU has it) and the scalar loop
    give the same int32 accumulators: random bytes (every nibble value, -8
    included), int8 activations over the whole range, and the extremes."""
    rng = np.random.default_rng(rows * 1000 + width)
    cases = [(rng.integers(0, 256, (rows, width // 2), dtype=np.uint8),
              rng.integers(-128, 128, width, dtype=np.int8)),
             (np.full((rows, width // 2), 0x88, np.uint8), np.full(width, -128, np.int8)),
             (np.full((rows, width // 2), 0x77, np.uint8), np.full(width, 127, np.int8))]
    try:
        for w, x in cases:
            oracle.set_simd(False)
            ref = oracle.int4_i8_gemv_acc(x, w, rows, width)
            oracle.set_simd(True)
            got = oracle.int4_i8_gemv_acc(x, w, rows, width)
            np.testing.assert_array_equal(got, ref)
            # and the closed form on the unpacked values (int64)
            lo = (w & 0xF).astype(np.int64)
            hi = (w >> 4).astype(np.int64)
            full = np.empty((rows, width), np.int64)
            full[:, 0::2] = np.where(lo > 7, lo - 16, lo)
            full[:, 1::2] = np.where(hi > 7, hi - 16, hi)
            np.testing.assert_array_equal(ref, full @ x.astype(np.int64))
    finally:
        oracle.set_simd(True)
