"""Pins the oracle's decode step (forward_token, cpu_lightspark.py:424-468 in
the reference repository) against golden vectors written by running the
reference's own forward_token (tests/golden/make_forward_golden.py)."""
import numpy as np
import pytest

import oracle

KEYS = ("qkv", "qkv_scales", "o", "o_scales", "gate_up", "gate_up_scales", "down",
        "down_scales", "input_norm", "post_norm", "q_norm", "k_norm")


def oracle_model(g):
    arrays = {k: [np.ascontiguousarray(a) for a in g[k]] for k in KEYS}
    for k in ("embedding", "embedding_scales", "final_norm", "rope_cos", "rope_sin"):
        arrays[k] = np.ascontiguousarray(g[k])
    return oracle.OracleModel(g["config"], arrays)


def test_forward_matches_reference_composition(forward_golden):
    g = forward_golden
    m = oracle_model(g)
    cap = g["keys"].shape[1]
    n = len(g["tokens"])
    st = m.new_state(cap, kv_f32=True)
    for i, t in enumerate(g["tokens"]):
        tok = m.forward_token(int(t), st)
        assert tok == g["greedy"][i]
        # only reduction order differs (qk-norm, softmax, exp): a few ulp
        np.testing.assert_allclose(st.logits, g["logits"][i], rtol=0, atol=2e-6)
    np.testing.assert_allclose(st.x, g["final_x"], rtol=0, atol=2e-6)
    np.testing.assert_allclose(st.keys[:, :n], g["keys"][:, :n], rtol=0, atol=2e-6)
    np.testing.assert_allclose(st.values[:, :n], g["values"][:, :n], rtol=0, atol=2e-6)


def test_forward_fp16_cache_stays_close(forward_golden):
    g = forward_golden
    m = oracle_model(g)
    n = len(g["tokens"])
    st = m.new_state(n)
    for i, t in enumerate(g["tokens"]):
        tok = m.forward_token(int(t), st)
        assert tok == g["greedy"][i]
        assert np.abs(st.logits - g["logits"][i]).max() < 0.1
    # the first token's keys see identical inputs, so they are the fp16 of the fp32 cache
    np.testing.assert_array_equal(st.keys[0, 0], g["keys"][0, 0].astype(np.float16).view(np.uint16))


def test_forward_errors(forward_golden):
    g = forward_golden
    m = oracle_model(g)
    st = m.new_state(1)
    with pytest.raises(ValueError, match="outside the vocabulary"):
        m.forward_token(g["config"]["vocab_size"], st)
    with pytest.raises(ValueError, match="outside the vocabulary"):
        m.forward_token(-1, st)
    m.forward_token(3, st)
    with pytest.raises(ValueError, match="capacity exhausted"):
        m.forward_token(3, st)


def test_embedding_row_decode(forward_golden):
    g = forward_golden
    m = oracle_model(g)
    t = 300
    w = oracle.unpack_int4(g["embedding"][t:t + 1], g["config"]["hidden_size"])[0]
    np.testing.assert_array_equal(m.embedding(t), w.astype(np.float32) * g["embedding_scales"][t])
