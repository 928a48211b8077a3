"""The reference's on-disk int4 cache (cpu_lightspark.py:556-686 in the
reference repository) read by harsh4b_amd.cache: layout, manifest checks,
fusion, norm weights, and a decode step of a model loaded from a cache
against the CPU oracle."""
import json

import numpy as np
import pytest

from harsh4b_amd import cache

KEYS = ("qkv", "qkv_scales", "o", "o_scales", "gate_up", "gate_up_scales", "down", "down_scales")
NORMS = ("input_norm", "post_norm", "q_norm", "k_norm")


def golden_cache(g, directory, **kw):
    arrays = {k: [np.asarray(a) for a in g[k]] for k in KEYS}
    single = cache.split_fused(g["config"], arrays)
    return cache.write_cache(directory, g["config"], single, g["embedding"], g["embedding_scales"], **kw)


def golden_norm_state(g):
    state = {}
    keys = cache.norm_keys(g["config"])
    for k in NORMS:
        for i, name in enumerate(keys[k]):
            state[name] = np.asarray(g[k][i], dtype=np.float32)
    state[keys["final_norm"]] = np.asarray(g["final_norm"], dtype=np.float32)
    return state


def test_projection_names_follow_reference_order():
    config = dict(num_hidden_layers=2)
    names = cache.projection_names(config)
    assert len(names) == 14
    assert names[:7] == ["model.layers.0.self_attn.q_proj", "model.layers.0.self_attn.k_proj",
                         "model.layers.0.self_attn.v_proj", "model.layers.0.self_attn.o_proj",
                         "model.layers.0.mlp.gate_proj", "model.layers.0.mlp.up_proj",
                         "model.layers.0.mlp.down_proj"]
    # the reference builds 252 names for Qwen3-4B (cpu_lightspark.py:597)
    from harsh4b_amd.config import QWEN3_4B
    assert len(cache.projection_names(QWEN3_4B)) == 252
    assert cache.slug("model.layers.3.mlp.up_proj") == "model_layers_3_mlp_up_proj"


def test_round_trip_files_and_fusion(forward_golden, tmp_path):
    g = forward_golden
    d = golden_cache(g, tmp_path / "c")
    manifest = json.loads((d / "manifest.json").read_text())
    name = "model.layers.1.self_attn.k_proj"
    assert manifest["projections"][name] == {"weights": "model_layers_1_self_attn_k_proj.int4.npy",
                                             "scales": "model_layers_1_self_attn_k_proj.scales.npy"}
    assert manifest["complete"] is True
    arrays = cache.read_cache(d, g["config"])
    for k in KEYS:
        for i in range(2):
            np.testing.assert_array_equal(arrays[k][i], g[k][i])
    np.testing.assert_array_equal(arrays["embedding"], g["embedding"])
    np.testing.assert_array_equal(arrays["embedding_scales"], g["embedding_scales"])
    # the fused qkv rows are q, then k, then v, each file the reference's shape
    k_w = np.load(d / "model_layers_1_self_attn_k_proj.int4.npy", allow_pickle=False)
    assert k_w.shape == (128, 64) and k_w.dtype == np.uint8
    np.testing.assert_array_equal(arrays["qkv"][1][256:384], k_w)


def test_manifest_checks(forward_golden, tmp_path):
    g = forward_golden
    d = golden_cache(g, tmp_path / "inc", complete=False)
    with pytest.raises(ValueError, match="incomplete"):
        cache.read_cache(d, g["config"])
    cache.read_cache(d, g["config"], allow_incomplete=True)
    bad = golden_cache(g, tmp_path / "fmt", identity={"format": "other", "embedding": cache.EMBEDDING_FORMAT})
    with pytest.raises(ValueError, match="format"):
        cache.read_cache(bad, g["config"])
    with pytest.raises(ValueError, match="no LiteSpark cache manifest"):
        cache.read_cache(tmp_path / "missing", g["config"])


def test_identity_must_match_checkpoint(forward_golden, tmp_path):
    g = forward_golden
    ckpt = tmp_path / "model.lat.pt"
    ckpt.write_bytes(b"checkpoint bytes")
    digest, identity = cache.cache_identity(ckpt)
    assert len(digest) == 16 and identity["size"] == 16 and identity["version"] == 2
    d = golden_cache(g, tmp_path / digest, identity=identity)
    cache.read_cache(d, g["config"], model_path=ckpt)
    ckpt.write_bytes(b"a different checkpoint")
    with pytest.raises(ValueError, match="does not match checkpoint"):
        cache.read_cache(d, g["config"], model_path=ckpt)


def test_shape_and_dtype_errors(forward_golden, tmp_path):
    g = forward_golden
    d = golden_cache(g, tmp_path / "c")
    np.save(d / "model_layers_0_mlp_down_proj.scales.npy", np.zeros(7, np.float32))
    with pytest.raises(ValueError, match="invalid LiteSpark cache shape for model.layers.0.mlp.down_proj"):
        cache.read_cache(d, g["config"])
    d2 = golden_cache(g, tmp_path / "c2")
    np.save(d2 / "embedding.int4.npy", np.zeros((512, 64), np.int8))
    with pytest.raises(ValueError, match="embedding"):
        cache.read_cache(d2, g["config"])


def test_pickled_npy_is_refused(forward_golden, tmp_path):
    g = forward_golden
    d = golden_cache(g, tmp_path / "c")
    np.save(d / "model_layers_0_self_attn_o_proj.int4.npy", np.array([{"a": 1}], dtype=object), allow_pickle=True)
    with pytest.raises(ValueError):
        cache.read_cache(d, g["config"])


def test_norms_from_state_dict_file(forward_golden, tmp_path):
    torch = pytest.importorskip("torch")
    g = forward_golden
    state = {k: torch.from_numpy(v.copy()) for k, v in golden_norm_state(g).items()}
    path = tmp_path / "norms.pt"
    torch.save(state, path)
    norms = cache.read_norms(path, g["config"])
    for k in NORMS:
        for i in range(2):
            np.testing.assert_array_equal(norms[k][i], g[k][i])
    np.testing.assert_array_equal(norms["final_norm"], g["final_norm"])
    del state["model.norm.weight"]
    with pytest.raises(ValueError, match="model.norm.weight is missing"):
        cache.read_norms(state, g["config"])


@pytest.mark.gpu
def test_model_from_cache_decodes_like_oracle(forward_golden, tmp_path):
    torch = pytest.importorskip("torch")
    import oracle
    from harsh4b_amd.synthetic import host_arrays
    from tests.gpu_util import assert_bits_equal, to_host
    g = forward_golden
    print("\n[gpu] cache -> device model, two golden tokens", flush=True)
    d = golden_cache(g, tmp_path / "c")
    model = cache.load_litespark_cache(d, golden_norm_state(g), config=g["config"])
    ref = oracle.OracleModel(g["config"], host_arrays(model))
    st, rs = model.new_state(4), ref.new_state(4)
    for i, t in enumerate(g["tokens"][:2]):
        logits = model.forward_token(int(t), st)
        tok = model.greedy_token(st)
        assert tok == ref.forward_token(int(t), rs) == int(g["greedy"][i])
        assert_bits_equal(to_host(logits), rs.logits, f"logits step {i}")
    st.check_status()
    torch.cuda.synchronize()


# ---- a cache written by the reference's own converter -----------------------------
# tests/golden/ref_cache/ was written by the reference's _convert_projection,
# _convert_embedding, _cache_identity and _atomic_json (cpu_lightspark.py:149-243,
# 574-610) on a 2-layer synthetic LATTICE model, and ref_cache_forward.npz holds the
# reference's forward_token logits over it (tests/golden/make_cache_golden.py).
from pathlib import Path  # noqa: E402

REF_CACHE = Path(__file__).resolve().parent / "golden" / "ref_cache"


@pytest.fixture(scope="module")
def ref_cache_golden():
    with np.load(REF_CACHE.parent / "ref_cache_forward.npz", allow_pickle=False) as f:
        g = {k: f[k] for k in f.files}
    g["config"] = json.loads(bytes(g["config_json"]).decode())
    g["identity"] = json.loads(bytes(g["identity_json"]).decode())
    g["norms"] = {str(name): g[f"norm_{i}"] for i, name in enumerate(g["norm_names"])}
    return g


def test_reference_written_cache_manifest_and_files(ref_cache_golden):
    g = ref_cache_golden
    manifest = cache.read_manifest(REF_CACHE)
    assert manifest["identity"] == g["identity"]
    # the reference's directory digest of that identity record
    assert cache.identity_digest(g["identity"]) == bytes(g["digest"]).decode()
    arrays = cache.read_cache(REF_CACHE, g["config"])
    # fused q|k|v and gate|up rows, each part the file the reference wrote
    q = np.load(REF_CACHE / "model_layers_1_self_attn_q_proj.int4.npy", allow_pickle=False)
    v = np.load(REF_CACHE / "model_layers_1_self_attn_v_proj.int4.npy", allow_pickle=False)
    np.testing.assert_array_equal(arrays["qkv"][1][:q.shape[0]], q)
    np.testing.assert_array_equal(arrays["qkv"][1][-v.shape[0]:], v)
    up = np.load(REF_CACHE / "model_layers_0_mlp_up_proj.scales.npy", allow_pickle=False)
    np.testing.assert_array_equal(arrays["gate_up_scales"][0][-up.shape[0]:], up)
    assert arrays["embedding"].shape == (512, 64) and arrays["embedding_scales"].dtype == np.float32


def test_oracle_on_reference_written_cache_matches_reference_forward(ref_cache_golden):
    import oracle
    g = ref_cache_golden
    arrays = {k: [np.ascontiguousarray(a) for a in v] if isinstance(v, list) else np.ascontiguousarray(v)
              for k, v in cache.read_cache(REF_CACHE, g["config"]).items()}
    arrays.update(cache.read_norms(g["norms"], g["config"]))
    arrays["rope_cos"], arrays["rope_sin"] = g["rope_cos"], g["rope_sin"]
    m = oracle.OracleModel(g["config"], arrays)
    st = m.new_state(len(g["tokens"]), kv_f32=True)
    for i, t in enumerate(g["tokens"]):
        assert m.forward_token(int(t), st) == g["greedy"][i]
        # only reduction order differs (qk-norm, softmax, exp): a few ulp
        np.testing.assert_allclose(st.logits, g["logits"][i], rtol=0, atol=2e-6)


@pytest.mark.gpu
def test_gpu_decode_from_reference_written_cache(ref_cache_golden):
    torch = pytest.importorskip("torch")
    import oracle
    from harsh4b_amd.synthetic import host_arrays
    from tests.gpu_util import assert_bits_equal, to_host
    g = ref_cache_golden
    print("\n[gpu] reference-written cache -> device model", flush=True)
    model = cache.load_litespark_cache(REF_CACHE, g["norms"], config=g["config"])
    ref = oracle.OracleModel(g["config"], host_arrays(model))
    n = len(g["tokens"])
    st, rs = model.new_state(n), ref.new_state(n)
    for i, t in enumerate(g["tokens"]):
        logits = model.forward_token(int(t), st)
        tok = model.greedy_token(st)
        assert tok == ref.forward_token(int(t), rs) == int(g["greedy"][i])
        assert_bits_equal(to_host(logits), rs.logits, f"logits step {i}")
    st.check_status()
    torch.cuda.synchronize()
