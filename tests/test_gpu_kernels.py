"""GPU parity of the HIP kernels against the CPU oracle (bit-exact), through
the C ABI of libhq.so.  Reference: cpu_kernels/litespark_int4.cpp and the
known-answer tests of tests/test_cpu_lightspark.py (reference repository)."""
import numpy as np
import pytest

import oracle
from tests.gpu_util import assert_bits_equal, dev, random_int4, to_dev, to_host

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(autouse=True)
def _announce(request):
    print(f"\n[gpu] {request.node.nodeid}", flush=True)
    yield
    torch.cuda.synchronize()


def lightspark():
    from harsh4b_amd import lightspark as ls
    return ls


# ------------------------------------------------------------------ GEMV
def test_gemv_known_answer(kat):
    ls = lightspark()
    w = kat["gemv_w"]
    p = ls.LiteSparkProjection(to_dev(oracle.pack_int4(w)), to_dev(kat["gemv_scales"]))
    out = ls.int4_i8_gemv(to_dev(kat["gemv_x"]), p, float(kat["gemv_act"]))
    got = to_host(out)
    np.testing.assert_allclose(got, kat["gemv_expected"], rtol=2e-6, atol=2e-5)
    ref = oracle.int4_i8_gemv(kat["gemv_x"], oracle.pack_int4(w), kat["gemv_scales"],
                              float(kat["gemv_act"]), w.shape[0], w.shape[1])
    assert_bits_equal(got, ref, "KAT gemv")


@pytest.mark.parametrize("rows,width", [(3, 30), (67, 130), (5, 2), (100, 96)])
def test_gemv_generic_path(rows, width):
    # widths that are not a multiple of 32 take the byte-load path
    ls = lightspark()
    rng = np.random.default_rng(rows + width)
    w = random_int4(rng, rows, width)
    x = rng.integers(-127, 128, size=width, dtype=np.int8)
    s = rng.random(rows, dtype=np.float32)
    p = ls.LiteSparkProjection(to_dev(oracle.pack_int4(w)), to_dev(s))
    got = to_host(ls.int4_i8_gemv(to_dev(x), p, 0.0123))
    assert_bits_equal(got, oracle.int4_i8_gemv(x, oracle.pack_int4(w), s, 0.0123, rows, width),
                      "generic gemv")


def test_gemv_unaligned_weights_take_generic_path():
    ls = lightspark()
    rng = np.random.default_rng(3)
    rows, width = 40, 256
    w = random_int4(rng, rows, width)
    packed = oracle.pack_int4(w)
    buf = torch.zeros(packed.size + 16, dtype=torch.uint8, device=dev())
    buf[1:1 + packed.size] = to_dev(packed.reshape(-1))
    x = rng.integers(-127, 128, size=width, dtype=np.int8)
    s = rng.random(rows, dtype=np.float32)
    out = torch.empty(rows, dtype=torch.float32, device=dev())
    from harsh4b_amd import _native
    xd, sd = to_dev(x), to_dev(s)      # keep both alive until the kernel has run
    _native.check(_native.lib().hq_int4_i8_gemv(xd.data_ptr(), buf.data_ptr() + 1, sd.data_ptr(),
                                                0.5, out.data_ptr(), rows, width, None), "gemv")
    assert_bits_equal(to_host(out), oracle.int4_i8_gemv(x, packed, s, 0.5, rows, width), "unaligned")


@pytest.mark.parametrize("rows,width", [(9728, 2560), (1001, 4096), (300, 20480), (7, 32768), (5000, 64)])
def test_gemv_int8_row_range_shapes(rows, width):
    # the reference-signature entry over the lane layouts of every width
    # class, rows that leave the last wave tile partly empty, and rows wider
    # than one batch of chunks per lane (32768: two batches)
    ls = lightspark()
    rng = np.random.default_rng(rows + 3 * width)
    w = random_int4(rng, rows, width)
    packed = oracle.pack_int4(w)
    x = rng.integers(-127, 128, size=width, dtype=np.int8)
    s = rng.uniform(0.005, 0.02, rows).astype(np.float32)
    p = ls.LiteSparkProjection(to_dev(packed), to_dev(s))
    got = to_host(ls.int4_i8_gemv(to_dev(x), p, 0.0071))
    assert_bits_equal(got, oracle.int4_i8_gemv(x, packed, s, 0.0071, rows, width), "row-range gemv")


QUANT_SHAPES = [(9728, 2560), (6144, 2560), (2560, 4096), (2560, 9728), (19456, 2560),
                (1000, 2560), (64, 64), (33, 10240), (8191, 4096)]


@pytest.mark.parametrize("rows,width", QUANT_SHAPES)
def test_quant_gemv_bit_exact(rows, width):
    ls = lightspark()
    rng = np.random.default_rng(rows * 7 + width)
    w = random_int4(rng, rows, width)
    packed = oracle.pack_int4(w)
    s = rng.uniform(0.005, 0.02, rows).astype(np.float32)
    x = rng.standard_normal(width).astype(np.float32)
    p = ls.LiteSparkProjection(to_dev(packed), to_dev(s))
    q = torch.empty(width, dtype=torch.int8, device=dev())
    act = torch.empty(1, dtype=torch.float32, device=dev())
    acc = torch.empty(rows, dtype=torch.int32, device=dev())
    out = ls.quant_int4_gemv(to_dev(x), p, q_out=q, act_out=act, acc_out=acc)
    r_out, r_q, r_act, r_acc = oracle.quant_int4_gemv(x, packed, s)
    assert_bits_equal(to_host(q), r_q, "q")
    assert_bits_equal(to_host(act), np.array([r_act], np.float32), "act")
    assert_bits_equal(to_host(acc), r_acc, "acc")
    assert_bits_equal(to_host(out), r_out, "out")
    # closed form: exact integer product of the same quantized vector
    np.testing.assert_array_equal(to_host(acc), w.astype(np.int64) @ r_q.astype(np.int64))


def test_quant_gemv_extremes():
    ls = lightspark()
    rows, width = 64, 9728
    w = np.full((rows, width), 7, dtype=np.int8)
    w[1::2] = -7
    x = np.full(width, 3.0, dtype=np.float32)
    x[::3] = -3.0
    packed = oracle.pack_int4(w)
    s = np.ones(rows, dtype=np.float32)
    p = ls.LiteSparkProjection(to_dev(packed), to_dev(s))
    acc = torch.empty(rows, dtype=torch.int32, device=dev())
    ls.quant_int4_gemv(to_dev(x), p, acc_out=acc)
    _, _, _, r_acc = oracle.quant_int4_gemv(x, packed, s)
    assert_bits_equal(to_host(acc), r_acc, "extreme acc")


def test_quant_gemv_zero_input():
    ls = lightspark()
    rows, width = 32, 2560
    rng = np.random.default_rng(0)
    packed = oracle.pack_int4(random_int4(rng, rows, width))
    p = ls.LiteSparkProjection(to_dev(packed), to_dev(np.ones(rows, np.float32)))
    act = torch.empty(1, dtype=torch.float32, device=dev())
    out = ls.quant_int4_gemv(torch.zeros(width, device=dev()), p, act_out=act)
    assert not to_host(out).any()
    assert to_host(act)[0] == np.float32(1e-5) / np.float32(127)


def test_quantize_and_rmsnorm_standalone():
    ls = lightspark()
    rng = np.random.default_rng(4)
    for n in (1, 255, 2560, 9728, 12345):
        x = (rng.standard_normal(n) * 5).astype(np.float32)
        g = rng.uniform(0.5, 1.5, n).astype(np.float32)
        q, act = ls.quantize_activation(to_dev(x))
        rq, ract = oracle.quantize_activation(x)
        assert_bits_equal(to_host(q), rq, f"quant n={n}")
        assert_bits_equal(to_host(act), np.array([ract], np.float32), f"act n={n}")
        y = ls.rmsnorm(to_dev(x), to_dev(g), 1e-6)
        assert_bits_equal(to_host(y), oracle.rmsnorm(x, g, 1e-6), f"rmsnorm n={n}")


# ------------------------------------------------------------------ attention
def test_gqa_known_answer(kat):
    ls = lightspark()
    kv, g, ctx, cap, d = (int(v) for v in kat["gqa_shape"])
    keys16 = kat["gqa_keys"].astype(np.float16)
    values16 = kat["gqa_values"].astype(np.float16)
    out = torch.empty((kv * g, d), dtype=torch.float32, device=dev())
    ls.gqa_decode(to_dev(kat["gqa_query"]), to_dev(keys16), to_dev(values16), out, ctx, kv, g, d)
    got = to_host(out)
    ref = oracle.gqa_decode_split(kat["gqa_query"], keys16.view(np.uint16), values16.view(np.uint16),
                                  ctx, kv, g, d)
    assert_bits_equal(got, ref, "gqa KAT vs oracle")
    # the reference's own expectation used fp32 K/V; fp16 storage moves it by < 2e-3
    np.testing.assert_allclose(got, kat["gqa_expected"], rtol=5e-3, atol=5e-3)


@pytest.mark.parametrize("ctx", [1, 2, 63, 64, 65, 129, 300, 4096, 4161, 9000])
def test_gqa_qwen_shape_bit_exact(ctx):
    ls = lightspark()
    rng = np.random.default_rng(ctx)
    kv, g, d = 8, 4, 128
    cap = ctx + 3
    q = rng.standard_normal((kv * g, d)).astype(np.float32)
    k16 = rng.standard_normal((cap, kv, d)).astype(np.float16)
    v16 = rng.standard_normal((cap, kv, d)).astype(np.float16)
    out = torch.empty((kv * g, d), dtype=torch.float32, device=dev())
    ls.gqa_decode(to_dev(q), to_dev(k16), to_dev(v16), out, ctx, kv, g, d)
    ref = oracle.gqa_decode_split(q, k16.view(np.uint16), v16.view(np.uint16), ctx, kv, g, d)
    assert_bits_equal(to_host(out), ref, f"gqa ctx={ctx}")


@pytest.mark.parametrize("d,g", [(16, 1), (32, 8), (64, 5), (128, 2)])
def test_gqa_other_head_shapes(d, g):
    ls = lightspark()
    rng = np.random.default_rng(d + g)
    kv, ctx = 3, 100
    q = rng.standard_normal((kv * g, d)).astype(np.float32)
    k16 = rng.standard_normal((ctx, kv, d)).astype(np.float16)
    v16 = rng.standard_normal((ctx, kv, d)).astype(np.float16)
    out = torch.empty((kv * g, d), dtype=torch.float32, device=dev())
    ls.gqa_decode(to_dev(q), to_dev(k16), to_dev(v16), out, ctx, kv, g, d)
    ref = oracle.gqa_decode_split(q, k16.view(np.uint16), v16.view(np.uint16), ctx, kv, g, d)
    assert_bits_equal(to_host(out), ref, f"gqa d={d} g={g}")


def test_gqa_repeated_calls_reuse_workspace():
    # one workspace serves every later call, longer or shorter (it holds
    # partials of earlier calls: each call writes every partial it reads)
    ls = lightspark()
    rng = np.random.default_rng(77)
    kv, g, d = 8, 4, 128
    for ctx in (500, 70, 500, 1):
        q = rng.standard_normal((kv * g, d)).astype(np.float32)
        k16 = rng.standard_normal((ctx, kv, d)).astype(np.float16)
        v16 = rng.standard_normal((ctx, kv, d)).astype(np.float16)
        out = torch.empty((kv * g, d), dtype=torch.float32, device=dev())
        ls.gqa_decode(to_dev(q), to_dev(k16), to_dev(v16), out, ctx, kv, g, d)
        ref = oracle.gqa_decode_split(q, k16.view(np.uint16), v16.view(np.uint16), ctx, kv, g, d)
        assert_bits_equal(to_host(out), ref, f"repeat ctx={ctx}")


def test_gqa_reference_call_values():
    # hq_gqa_decode called through the C ABI with exactly the integers the
    # reference's _attention passes (cpu_lightspark.py:394-406): context =
    # position + 1, kv_heads, groups, head_dim, score_stride = state.capacity,
    # on one layer of a [layers, capacity, kv_heads, head_dim] cache
    import ctypes
    from harsh4b_amd import _native
    lib = _native.lib()
    rng = np.random.default_rng(405)
    layers, capacity, kv, g, d = 3, 300, 8, 4, 128
    keys = rng.standard_normal((layers, capacity, kv, d)).astype(np.float16)
    values = rng.standard_normal((layers, capacity, kv, d)).astype(np.float16)
    kd, vd = to_dev(keys), to_dev(values)
    ws = torch.zeros(lib.hq_gqa_workspace_bytes(capacity, kv, g, d), dtype=torch.uint8, device=dev())
    for layer, position in ((0, 0), (2, 137), (1, capacity - 1)):
        end = position + 1
        q = rng.standard_normal((kv * g, d)).astype(np.float32)
        out = torch.empty((kv * g, d), dtype=torch.float32, device=dev())
        status = lib.hq_gqa_decode(to_dev(q).data_ptr(), kd[layer].data_ptr(), vd[layer].data_ptr(),
                                   ws.data_ptr(), out.data_ptr(), end, kv, g, d, capacity,
                                   ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert status == 0
        ref = oracle.gqa_decode_split(q, keys[layer].view(np.uint16), values[layer].view(np.uint16), end,
                                      kv, g, d)
        assert_bits_equal(to_host(out), ref, f"gqa layer={layer} end={end}")


# ------------------------------------------------------------------ argmax
def test_device_argmax_order(kat):
    ls = lightspark()
    assert ls.argmax(to_dev(kat["argmax_logits"])) == int(kat["argmax_expected"])
    rng = np.random.default_rng(5)
    x = rng.standard_normal(151936).astype(np.float32)
    x[[70000, 9000, 150000]] = 9.0
    assert ls.argmax(to_dev(x)) == int(np.argmax(x)) == 9000
    x[123456] = np.nan
    x[140000] = np.nan
    assert ls.argmax(to_dev(x)) == int(np.argmax(x)) == 123456
    assert ls.argmax(to_dev(np.array([-0.0, 0.0], np.float32))) == 0


# ------------------------------------------------------------------ sampler
def check_sample(logits, generated, rp, temperature, top_k, top_p, u, what):
    ls = lightspark()
    got = ls.sample_token(to_dev(logits), generated, rp, temperature, top_k, top_p, u)
    want = oracle.sample_token(logits, generated, rp, temperature, top_k, top_p, u)
    np.testing.assert_array_equal(got[1], want[1], err_msg=f"ids {what}")
    assert_bits_equal(got[2], want[2], f"probabilities {what}")
    assert got[0] == want[0], what
    return got


def test_sampler_reference_policy():
    # the reference runner's defaults (temperature 0.7, top-k 40, top-p 0.9,
    # repetition penalty 1.08) on Qwen3-4B's vocabulary
    rng = np.random.default_rng(11)
    for trial in range(12):
        logits = (rng.standard_normal(151936) * rng.uniform(1, 6)).astype(np.float32)
        generated = [int(t) for t in rng.integers(0, 151936, 40)]
        generated += generated[:5]                                  # repeats count once
        generated += [int(i) for i in np.argsort(-logits)[:8]]      # penalise some of the top
        check_sample(logits, generated, 1.08, 0.7, 40, 0.9, float(rng.random()), f"trial {trial}")


@pytest.mark.parametrize("n,top_k", [(151936, 1), (151936, 64), (151936, 107), (151936, 108), (151936, 500),
                                     (151936, 2048), (4096, 40), (4097, 40), (4097, 2048), (10, 40), (5, 5),
                                     (1, 3), (70000, 1500)])
def test_sampler_sizes_and_merge_rounds(n, top_k):
    rng = np.random.default_rng(n + top_k)
    logits = (rng.standard_normal(n) * 3).astype(np.float32)
    for u in (0.0, float(rng.random()), 0.999999):
        for top_p in (1.0, 0.9, 0.3):
            check_sample(logits, [0, n - 1], 1.3, 1.1, top_k, top_p, u, f"n={n} k={top_k} u={u} p={top_p}")


def test_sampler_ties_signs_and_penalty():
    rng = np.random.default_rng(3)
    # values on a coarse grid: long runs of equal values rank by index
    logits = (np.round(rng.standard_normal(151936) * 8) / 4).astype(np.float32)
    for top_k in (40, 300, 2048):
        check_sample(logits, [], 1.0, 1.0, top_k, 0.95, 0.37, f"ties k={top_k}")
    # -0/+0, infinities, negative logits under the penalty, a tiny top-p
    x = rng.standard_normal(50000).astype(np.float32) - 4
    x[[10, 11, 12]] = [0.0, -0.0, 0.0]
    x[[20, 21]] = -np.inf
    gen = [int(i) for i in np.argsort(-x)[:30]] + [10, 11, 20]
    check_sample(x, gen, 1.5, 0.5, 64, 0.9, 0.61, "signs")
    check_sample(x, gen, 1.5, 0.5, 64, 1e-6, 0.99, "tiny top-p")
    small = np.array([0.5, 3.0, -2.0, 2.9, 1.0], np.float32)
    assert check_sample(small, [1, 1, 1], 2.0, 1.0, 5, 1.0, 0.0, "small")[0] == 3
    assert check_sample(small, [], 1.0, 0.7, 1, 0.9, 0.999, "k=1")[0] == 1


def test_sampler_long_history_and_penalty_below_one():
    # 5000 generated ids (repeats included) spread over every 4096-logit
    # slice; a penalty below 1 raises positive logits and lowers negative ones
    rng = np.random.default_rng(17)
    logits = (rng.standard_normal(151936) * 3).astype(np.float32)
    generated = [int(t) for t in rng.integers(0, 151936, 4000)]
    generated += generated[:1000]
    for rp, k, p in ((1.08, 40, 0.9), (0.9, 64, 0.95), (1.5, 500, 1.0)):
        check_sample(logits, generated, rp, 0.8, k, p, float(rng.random()), f"rp={rp} k={k}")


def test_sample_logits_follows_the_generator():
    # sample_logits consumes the generator as Generator.choice does: one
    # random() per token, so the device run and the oracle draw the same u
    ls = lightspark()

    class Args:
        argmax, repetition_penalty, temperature, top_k, top_p = False, 1.08, 0.7, 40, 0.9
    rng = np.random.default_rng(2)
    g_dev, g_ref = np.random.default_rng(0), np.random.default_rng(0)
    generated = []
    for step in range(20):
        logits = (rng.standard_normal(151936) * 2).astype(np.float32)
        token = ls.sample_logits(to_dev(logits), generated, Args(), g_dev)
        want = oracle.sample_token(logits, generated, 1.08, 0.7, 40, 0.9, g_ref.random())[0]
        assert token == want, step
        generated.append(token)
    assert g_dev.random() == g_ref.random()
    with pytest.raises(ValueError, match="top_k"):
        ls.sample_token(to_dev(logits), [], 1.0, 1.0, 4096, 1.0, 0.5)
    with pytest.raises(IndexError):
        ls.sample_token(to_dev(logits), [151936], 1.08, 1.0, 4, 1.0, 0.5)


# ------------------------------------------------------------------ batched
@pytest.mark.parametrize("m", [1, 8, 16, 32, 40])
@pytest.mark.parametrize("rows,width", [(2560, 9728), (6144, 2560), (2560, 4096), (19456, 2560), (100, 96)])
def test_batched_gemm_bit_exact(m, rows, width):
    # Qwen3-4B's down, qkv, o and gate_up shapes (rows staged through LDS)
    # and a ragged one
    ls = lightspark()
    rng = np.random.default_rng(m * 31 + rows)
    w = random_int4(rng, rows, width)
    packed = oracle.pack_int4(w)
    s = rng.uniform(0.005, 0.02, rows).astype(np.float32)
    x = rng.standard_normal((m, width)).astype(np.float32)
    p = ls.LiteSparkProjection(to_dev(packed), to_dev(s))
    acc = torch.empty((m, rows), dtype=torch.int32, device=dev())
    qo = torch.empty((m, width), dtype=torch.int8, device=dev())
    ao = torch.empty(m, dtype=torch.float32, device=dev())
    out = ls.quant_int4_gemm(to_dev(x), p, q_out=qo, act_out=ao, acc_out=acc)
    ref_out = np.empty((m, rows), np.float32)
    ref_acc = np.empty((m, rows), np.int32)
    for i in range(m):
        o, q, a, c = oracle.quant_int4_gemv(x[i], packed, s)
        ref_out[i], ref_acc[i] = o, c
    assert_bits_equal(to_host(acc), ref_acc, "batched acc")
    assert_bits_equal(to_host(out), ref_out, "batched out")
    # the int8 entry with the quantized inputs gives the same result
    out2 = ls.int4_i8_gemm(qo, ao, p)
    assert_bits_equal(to_host(out2), ref_out, "int8 entry")
    # and equals m independent batch-1 GEMVs
    for i in (0, m - 1):
        one = ls.int4_i8_gemv(qo[i].contiguous(), p, float(to_host(ao)[i]))
        assert_bits_equal(to_host(one), ref_out[i], f"gemv row {i}")


@pytest.mark.parametrize("m", [3, 17])
def test_batched_gemm_wide_rows(m):
    # rows wider than 10240 columns take the kernel with MFMA-shaped loads
    ls = lightspark()
    rng = np.random.default_rng(900 + m)
    rows, width = 72, 10496
    w = random_int4(rng, rows, width)
    packed = oracle.pack_int4(w)
    s = rng.uniform(0.005, 0.02, rows).astype(np.float32)
    q = rng.integers(-127, 128, (m, width)).astype(np.int8)
    a = rng.uniform(0.001, 0.01, m).astype(np.float32)
    p = ls.LiteSparkProjection(to_dev(packed), to_dev(s))
    acc = torch.empty((m, rows), dtype=torch.int32, device=dev())
    out = ls.int4_i8_gemm(to_dev(q), to_dev(a), p, acc_out=acc)
    assert_bits_equal(to_host(acc), oracle.int4_i8_gemm_acc(q, packed, rows, width), "wide acc")
    ref = np.stack([oracle.int4_i8_gemv(q[i], packed, s, a[i], rows, width) for i in range(m)])
    assert_bits_equal(to_host(out), ref, "wide out")
