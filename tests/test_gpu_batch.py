"""GPU parity of the batched decode step (hq_decode_batch): M independent
sequences stepped together must give, for every sequence, the bits M
separate forward_token steps give (cpu_lightspark.py:424-468 in the
reference repository, applied to each sequence): logits, greedy tokens, the
K/V rows written, the residual and the position; and the oracle's logits."""
import numpy as np
import pytest

import oracle
from tests.gpu_util import assert_bits_equal, to_dev, to_host

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

KEYS = ("qkv", "qkv_scales", "o", "o_scales", "gate_up", "gate_up_scales", "down",
        "down_scales", "input_norm", "post_norm", "q_norm", "k_norm")


@pytest.fixture(autouse=True)
def _announce(request):
    print(f"\n[gpu] {request.node.nodeid}", flush=True)
    yield
    torch.cuda.synchronize()


def golden_model(g):
    from harsh4b_amd.synthetic import model_from_arrays
    arrays = {k: [np.ascontiguousarray(a) for a in g[k]] for k in KEYS}
    for k in ("embedding", "embedding_scales", "final_norm"):
        arrays[k] = np.ascontiguousarray(g[k])
    return model_from_arrays(g["config"], arrays)


def _compare(model, batched, single, tag):
    """Batched states against single-step states: positions, tokens, logits,
    residual and every K/V row written so far, bit for bit."""
    for i, (a, b) in enumerate(zip(batched, single)):
        assert a.position == b.position, (tag, i)
        assert int(a.device_position.item()) == int(b.device_position.item()) == a.position, (tag, i)
        assert model.greedy_token(a) == model.greedy_token(b), (tag, i)
        assert_bits_equal(to_host(a.logits), to_host(b.logits), f"{tag} logits {i}")
        assert_bits_equal(to_host(a.x), to_host(b.x), f"{tag} residual {i}")
        n = a.position
        assert_bits_equal(to_host(a.keys)[:, :n].view(np.uint16), to_host(b.keys)[:, :n].view(np.uint16),
                          f"{tag} keys {i}")
        assert_bits_equal(to_host(a.values)[:, :n].view(np.uint16), to_host(b.values)[:, :n].view(np.uint16),
                          f"{tag} values {i}")
        a.check_status()
        b.check_status()


def test_tiny_model_batch_matches_single_steps_and_oracle(forward_golden):
    g = forward_golden
    model = golden_model(g)
    toks = [int(t) for t in g["tokens"]]
    histories = [[], toks[:1], toks[:3], toks[:6]]
    nxt = [toks[0], toks[2], toks[4], toks[1]]
    cap = 12
    A = [model.new_state(cap) for _ in histories]
    B = [model.new_state(cap) for _ in histories]
    for st_a, st_b, h in zip(A, B, histories):
        for t in h:
            model.forward_token(t, st_a)
            model.forward_token(t, st_b)
    model.forward_tokens(nxt, A)
    for t, st in zip(nxt, B):
        model.forward_token(t, st)
    _compare(model, A, B, "tiny step")
    # the oracle, sequence by sequence
    from harsh4b_amd.synthetic import host_arrays
    ref = oracle.OracleModel(model.config, host_arrays(model))
    for i, (h, t) in enumerate(zip(histories, nxt)):
        rs = ref.new_state(cap)
        for u in h + [t]:
            ref.forward_token(u, rs)
        assert_bits_equal(to_host(A[i].logits), rs.logits, f"oracle logits {i}")
    # then three batched greedy steps from a captured graph against
    # decode_greedy on each single state
    model.decode_greedy_batch(A, 3)
    for st in B:
        model.decode_greedy(st, 3)
    _compare(model, A, B, "tiny greedy")


def test_batch_rejects_bad_input(forward_golden):
    g = forward_golden
    model = golden_model(g)
    st = model.new_state(2)
    with pytest.raises(ValueError, match="one token per"):
        model.forward_tokens([1, 2], [st])
    with pytest.raises(ValueError, match="twice"):
        model.forward_tokens([1, 2], [st, st])
    with pytest.raises(ValueError, match="outside the vocabulary"):
        model.forward_tokens([int(g["config"]["vocab_size"])], [st])
    with pytest.raises(ValueError, match="1 to 32"):
        model.forward_tokens([], [])


@pytest.fixture(scope="module")
def qwen():
    from harsh4b_amd.config import QWEN3_4B
    from harsh4b_amd.synthetic import random_model
    model = random_model(QWEN3_4B, seed=11)
    torch.cuda.synchronize()
    return model


@pytest.mark.parametrize("m,big", [(8, False), (32, False), (8, True), (16, False), (16, True), (1, False)])
def test_qwen3_4b_batch_matches_single_steps(qwen, m, big):
    # M sequences with histories of 1 .. 300 positions (one to five chunks
    # of attention, one to two chunk groups), stepped together and alone
    # (up to 8 sequences the qkv GEMM runs in the attention's launch, from
    # 9 on one attention block per sequence and kv head); with `big` one
    # state holds 600 positions (more than eight chunks: the split attention
    # whose blocks walk further splits and whose tails combine the chunk
    # partials in batches of eight)
    model = qwen
    rng = np.random.default_rng(100 + m)
    lengths = [int(v) for v in rng.integers(1, 300, m)]
    lengths[0], lengths[-1] = 1, 300
    prompts = [[int(t) for t in rng.integers(0, 151936, n)] for n in lengths]
    A, B = [], []
    for i, pr in enumerate(prompts):
        for group in (A, B):
            st = model.new_state(600 if big and i == 1 else len(pr) + 4)
            model.prefill(pr, st)
            group.append(st)
    nxt = [int(t) for t in rng.integers(0, 151936, m)]
    model.forward_tokens(nxt, A)
    for t, st in zip(nxt, B):
        model.forward_token(t, st)
    _compare(model, A, B, f"M={m} step")
    model.decode_greedy_batch(A, 2)
    for st in B:
        model.decode_greedy(st, 2)
    _compare(model, A, B, f"M={m} greedy")


def _step_counter(model, cap):
    """The batched workspace's step counter (its first 4 bytes)."""
    return model._batch_workspaces[cap][:4].view(torch.int32)


def test_qwen3_4b_batch_step_counter_wrap(qwen):
    # A step accepts only the values its own launches tagged: an M = 16 step
    # leaves tagged values in rows 0-15; the counter is then set two short of
    # its period, an M = 8 step runs at the last count, and the next M = 16
    # step wraps: it must clear the old rows 8-15 (tagged at count 1, the
    # count the wrap restarts at) before any launch waits on them.  Then the
    # workspace is zero-filled with its counter set to 2^23 (outside the
    # period), and an M = 8 and an M = 16 step run from it.  Every step equals M single
    # steps bit for bit.  (Before the counter had a period, a tag older than
    # 2^23 steps counted as current.)
    period = 1 << 23
    model = qwen
    rng = np.random.default_rng(23)
    cap = 96
    model._batch_workspaces.pop(cap, None)   # a fresh zero-filled workspace
    lengths = [1, 70, 5, 33, 64, 2, 9, 80, 17, 3, 65, 40, 12, 7, 50, 26]
    A, B = [], []
    for n in lengths:
        pr = [int(t) for t in rng.integers(0, 151936, n)]
        for group in (A, B):
            st = model.new_state(cap)
            model.prefill(pr, st)
            group.append(st)

    def step(m, tag):
        nxt = [int(t) for t in rng.integers(0, 151936, m)]
        model.forward_tokens(nxt, A[:m])
        for t, st in zip(nxt, B[:m]):
            model.forward_token(t, st)
        _compare(model, A[:m], B[:m], tag)

    step(16, "count 1")
    ctr = _step_counter(model, cap)
    assert int(ctr.item()) == 1
    ctr.fill_(period - 2)
    step(8, "last count")
    assert int(_step_counter(model, cap).item()) == period - 1
    step(16, "wrap")
    assert int(_step_counter(model, cap).item()) == 1
    step(8, "after wrap")
    assert int(_step_counter(model, cap).item()) == 2

    # a zero-filled workspace whose counter reads 2^23 (outside the period)
    ws = model._batch_workspaces[cap]
    ws.zero_()
    _step_counter(model, cap).fill_(period)
    step(8, "outside the period, M = 8")
    assert int(_step_counter(model, cap).item()) == 1
    step(16, "outside the period, M = 16")
    assert int(_step_counter(model, cap).item()) == 2


@pytest.mark.parametrize("m", [8, 32])
def test_qwen3_4b_batch_full_state_spares_the_rest(qwen, m):
    # One sequence of the batch sits at its cache's capacity on the device
    # (the host's capacity check passed, as a C-ABI caller's could): its
    # status gets HQ_STEP_FULL and it writes no K/V row, and every other
    # sequence's step equals its single step bit for bit (M = 8: the qkv
    # GEMM and the attention in one launch; M = 32: one attention block per
    # sequence and kv head).
    from harsh4b_amd import _native
    model = qwen
    rng = np.random.default_rng(700 + m)
    lengths = [int(v) for v in rng.integers(1, 200, m)]
    lengths[0] = 64
    A, B = [], []
    for n in lengths:
        pr = [int(t) for t in rng.integers(0, 151936, n)]
        for group in (A, B):
            st = model.new_state(n + 4)
            model.prefill(pr, st)
            group.append(st)
    full = 3
    A[full].device_position.fill_(A[full].capacity)
    keys0, values0 = to_host(A[full].keys).copy(), to_host(A[full].values).copy()
    nxt = [int(t) for t in rng.integers(0, 151936, m)]
    model.forward_tokens(nxt, A)
    for t, st in zip(nxt, B):
        model.forward_token(t, st)
    A[full].synchronize()
    assert int(A[full].status.item()) & _native.HQ_STEP_FULL
    assert_bits_equal(to_host(A[full].keys).view(np.uint16), keys0.view(np.uint16), "full state's keys")
    assert_bits_equal(to_host(A[full].values).view(np.uint16), values0.view(np.uint16), "full state's values")
    keep = [i for i in range(m) if i != full]
    _compare(model, [A[i] for i in keep], [B[i] for i in keep], f"M={m} beside a full state")


@pytest.fixture(scope="module")
def qwen_oracle(qwen):
    from harsh4b_amd.synthetic import host_arrays
    return oracle.OracleModel(qwen.config, host_arrays(qwen))


@pytest.mark.parametrize("m,cap", [(8, 512), (16, 512), (32, 512), (8, 700)])
def test_qwen3_4b_batch_matches_oracle(qwen, qwen_oracle, m, cap):
    # The full-size batched step against the oracle directly, sequence by
    # sequence (8 KV heads x 4 query heads, hidden 2560): each sequence gets
    # its own N(0,1) fp16 cache of a ragged length (0 .. cap - 2 positions,
    # chunk edges included), then one batched step with given tokens and one
    # greedy batched step.  M = 8 and 16 run the qkv GEMM inside the
    # attention's launch, M = 32 apart from it; capacity 512 keeps the
    # attention's combine in the launch tails (at most 8 chunks), 700 sends
    # it through the combine kernel.  Logits, greedy tokens and the K/V rows
    # written must equal the oracle's bits.
    model, ref = qwen, qwen_oracle
    rng = np.random.default_rng(5000 + m + cap)
    contexts = [int(v) for v in rng.integers(0, cap - 2, m)]
    edges = [0, 1, 63, 64, 65, cap - 2]
    contexts[:len(edges)] = edges[:m]
    layers, kv, d = model.config["num_hidden_layers"], model.config["num_key_value_heads"], 128
    base = {name: rng.standard_normal((layers, cap + 2 * m, kv, d)).astype(np.float16) for name in ("keys", "values")}
    A, R = [], []
    for i, ctx in enumerate(contexts):
        st = model.new_state(cap)
        rs = ref.new_state(cap)
        for name in ("keys", "values"):
            cache = base[name][:, 2 * i:2 * i + ctx]
            getattr(st, name)[:, :ctx] = to_dev(cache)
            getattr(rs, name)[:, :ctx] = cache.view(np.uint16)
        st.device_position.fill_(ctx)
        st.position = ctx
        rs.position = ctx
        A.append(st)
        R.append(rs)
    torch.cuda.synchronize()
    toks = [int(t) for t in rng.integers(0, 151936, m)]
    for step in range(2):
        if step == 0:
            model.forward_tokens(toks, A)
        else:
            model.decode_greedy_batch(A, 1, use_graph=False)
        for i, (st, rs) in enumerate(zip(A, R)):
            rtok = ref.forward_token(toks[i], rs)
            tag = f"M={m} cap={cap} step {step} seq {i} ctx {contexts[i] + step}"
            assert_bits_equal(to_host(st.logits), rs.logits, f"{tag} logits")
            assert model.greedy_token(st) == rtok, tag
            p = contexts[i] + step
            assert_bits_equal(to_host(st.keys).view(np.uint16)[:, p], rs.keys[:, p], f"{tag} keys")
            assert_bits_equal(to_host(st.values).view(np.uint16)[:, p], rs.values[:, p], f"{tag} values")
            toks[i] = rtok
        for st in A:
            st.check_status()
