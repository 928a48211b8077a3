"""A tiny int4 cache written by the reference's own converter, and the
reference's forward_token logits over it.

The reference converts a LATTICE checkpoint once into its on-disk int4 cache
(cpu_lightspark.py:149-243 and :556-686 in the reference repository):
``_convert_projection`` reconstructs each projection from its LATTICE codes,
rotates it and row-quantizes it to int4, ``_convert_embedding`` quantizes the
tied embedding, and ``build_litespark_cpu`` writes ``manifest.json`` with the
``_cache_identity`` record.  ``build_litespark_cpu`` itself cannot run here
(it needs the absent third-party ``litespark_inference`` kernel and a real
checkpoint), so this script drives the same steps on a 2-layer synthetic
model: it calls the reference's ``_convert_projection`` on synthetic
LATTICE-coded projections, ``_convert_embedding`` on a random fp32 embedding,
and writes the manifest with the reference's ``_cache_identity`` and
``_atomic_json`` in the layout ``build_litespark_cpu`` uses.  It then loads
that cache the way ``build_litespark_cpu`` does (np.load of every file, q/k/v
and gate/up concatenated) and runs the reference's ``LiteSparkQwen.forward_token``
over a few tokens, with the same stand-in kernel as make_forward_golden.py
(the third-party quantize / RMSNorm / add / LM-head steps as this
repository's CPU oracle implements the spec).

Output: tests/golden/ref_cache/ (the cache directory, as the reference wrote
it) and tests/golden/ref_cache_forward.npz (norm weights, rope tables, tokens,
the reference's logits and greedy tokens, the identity record and digest).
Run:    python tests/golden/make_cache_golden.py [/path/to/reference]
"""
import json
import shutil
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
CACHE_DIR = HERE / "ref_cache"
OUT = HERE / "ref_cache_forward.npz"

CONFIG = {
    "hidden_size": 128, "intermediate_size": 256, "num_attention_heads": 2,
    "num_key_value_heads": 1, "head_dim": 128, "num_hidden_layers": 2,
    "vocab_size": 512, "rms_norm_eps": 1e-6, "rope_theta": 1000000,
    "max_position_embeddings": 64,
}
PROMPT = [9, 400, 77, 3]
DECODE_STEPS = 4
BLOCKSIZE = 16
SPLITS = {128: (8, 16), 256: (16, 16)}      # KOTMS rotation sizes: dim_l * dim_r = width


class Stored:
    """A checkpoint tensor stand-in: the reference reads LATTICE fields with .numpy()."""

    def __init__(self, array):
        self.array = np.ascontiguousarray(array)

    def numpy(self):
        return self.array


def lattice_projection(rng, rows, width, pack_codes):
    """Synthetic LATTICE fields of one projection in the layout
    _convert_projection reads (mask IDs 0-3 per weight, 2-bit T0 codes, compact
    T1 codes for the second-order weights (mask ID < 2), per-(mode, row, block)
    mu/a0/a1), and its two rotation matrices."""
    blocks = width // BLOCKSIZE
    maskid = rng.integers(0, 4, size=(rows, width), dtype=np.uint8)
    t0 = rng.integers(0, 4, size=(rows, width), dtype=np.uint8)
    second = maskid < 2
    n_t1 = int(second.sum())
    t1_flat = rng.integers(0, 4, size=n_t1, dtype=np.uint8)
    pad = (-n_t1) % 4
    t1c = np.pad(t1_flat, (0, pad))
    t1c = (t1c[0::4] | (t1c[1::4] << 2) | (t1c[2::4] << 4) | (t1c[3::4] << 6)).astype(np.uint8)
    packed = {
        "shape": (rows, width), "blocksize": BLOCKSIZE,
        "maskid": Stored(pack_codes(maskid)), "T0": Stored(pack_codes(t0)),
        "T1c": Stored(t1c), "n_T1": n_t1,
        "mu": Stored(rng.normal(0.0, 0.02, size=(4, rows, blocks)).astype(np.float32)),
        "a0": Stored(rng.uniform(0.005, 0.05, size=(4, rows, blocks)).astype(np.float32)),
        "a1": Stored(rng.uniform(0.002, 0.02, size=(2, rows, blocks)).astype(np.float32)),
        "o2_idx": Stored(np.array([0, 1], dtype=np.int64)),
    }
    dim_l, dim_r = SPLITS[width]
    left = Stored(rng.normal(0.0, 1.0 / np.sqrt(dim_l), size=(dim_l, dim_l)).astype(np.float32))
    right = Stored(rng.normal(0.0, 1.0 / np.sqrt(dim_r), size=(dim_r, dim_r)).astype(np.float32))
    return packed, left, right


def main(reference_root: str) -> None:
    sys.path.insert(0, str(REPO))
    sys.path.insert(0, reference_root)
    import oracle  # noqa: E402  (the spec functions of the stand-in kernel)
    import cpu_lightspark as ref
    from MLX.lattice_model import pack_codes

    class SpecKernel:
        """Stand-in for litespark_inference.torchless.kernel."""

        @staticmethod
        def rmsnorm_into(x, gamma, out, eps):
            out[:] = oracle.rmsnorm(x, gamma, eps)

        @staticmethod
        def quantize_activation(values, quantized):
            q, scale = oracle.quantize_activation(values)
            quantized[:] = q
            return float(scale)

        @staticmethod
        def add_inplace(x, y):
            np.add(x, y, out=x)

        @staticmethod
        def lm_head_int4(weights, scales, values, out, input_size):
            q, scale = oracle.quantize_activation(values)
            out[:] = oracle.int4_i8_gemv(q, weights, scales, scale, weights.shape[0], input_size)

    c = CONFIG
    H, I = c["hidden_size"], c["intermediate_size"]
    d, nq, nkv = c["head_dim"], c["num_attention_heads"], c["num_key_value_heads"]
    shapes = {"q_proj": (nq * d, H), "k_proj": (nkv * d, H), "v_proj": (nkv * d, H), "o_proj": (H, nq * d),
              "gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)}
    rng = np.random.default_rng(4096)
    if CACHE_DIR.exists():
        shutil.rmtree(CACHE_DIR)
    CACHE_DIR.mkdir(parents=True)
    # the checkpoint the identity record names: a stand-in file (its path and
    # mtime make the record machine-specific; the digest is kept with it)
    stub = CACHE_DIR / "checkpoint_stand_in.txt"
    stub.write_bytes(b"synthetic LATTICE checkpoint stand-in\n")
    digest, identity = ref._cache_identity(stub)
    manifest = {"identity": identity, "complete": False, "projections": {}}
    ref._atomic_json(CACHE_DIR / "manifest.json", manifest)
    names = []
    for index in range(c["num_hidden_layers"]):
        for block, proj in (("self_attn", "q_proj"), ("self_attn", "k_proj"), ("self_attn", "v_proj"),
                            ("self_attn", "o_proj"), ("mlp", "gate_proj"), ("mlp", "up_proj"),
                            ("mlp", "down_proj")):
            names.append((f"model.layers.{index}.{block}.{proj}", shapes[proj]))
    for name, (rows, width) in names:
        packed, left, right = lattice_projection(rng, rows, width, pack_codes)
        slug = name.replace(".", "_")
        wpath, spath = CACHE_DIR / f"{slug}.int4.npy", CACHE_DIR / f"{slug}.scales.npy"
        ref._convert_projection(packed, left, right, wpath, spath)
        manifest["projections"][name] = {"weights": wpath.name, "scales": spath.name}
        ref._atomic_json(CACHE_DIR / "manifest.json", manifest)
    embedding_src = rng.normal(0.0, 0.05, size=(c["vocab_size"], H)).astype(np.float32)
    ref._convert_embedding(embedding_src, CACHE_DIR / "embedding.int4.npy", CACHE_DIR / "embedding.scales.npy")
    manifest["complete"] = True
    ref._atomic_json(CACHE_DIR / "manifest.json", manifest)

    # norm weights (checkpoint tensors, not part of the cache)
    norms = {}
    for index in range(c["num_hidden_layers"]):
        p = f"model.layers.{index}"
        norms[f"{p}.input_layernorm.weight"] = rng.uniform(0.5, 1.5, size=H).astype(np.float32)
        norms[f"{p}.post_attention_layernorm.weight"] = rng.uniform(0.5, 1.5, size=H).astype(np.float32)
        norms[f"{p}.self_attn.q_norm.weight"] = rng.uniform(0.5, 1.5, size=d).astype(np.float32)
        norms[f"{p}.self_attn.k_norm.weight"] = rng.uniform(0.5, 1.5, size=d).astype(np.float32)
    norms["model.norm.weight"] = rng.uniform(0.5, 1.5, size=H).astype(np.float32)

    # the model as build_litespark_cpu assembles it from the cache (:619-662)
    def projection(name):
        files = manifest["projections"][name]
        return ref.LiteSparkProjection(np.load(CACHE_DIR / files["weights"], allow_pickle=False),
                                       np.load(CACHE_DIR / files["scales"], allow_pickle=False))

    def combine(*items):
        return ref.LiteSparkProjection(np.concatenate([i.weights for i in items], axis=0),
                                       np.concatenate([i.scales for i in items]))

    layers = []
    for index in range(c["num_hidden_layers"]):
        p = f"model.layers.{index}"
        attn, mlp = f"{p}.self_attn", f"{p}.mlp"
        layers.append(ref.QwenLayer(
            qkv=combine(projection(f"{attn}.q_proj"), projection(f"{attn}.k_proj"), projection(f"{attn}.v_proj")),
            o=projection(f"{attn}.o_proj"),
            gate_up=combine(projection(f"{mlp}.gate_proj"), projection(f"{mlp}.up_proj")),
            down=projection(f"{mlp}.down_proj"),
            input_norm=norms[f"{p}.input_layernorm.weight"],
            post_norm=norms[f"{p}.post_attention_layernorm.weight"],
            q_norm=norms[f"{attn}.q_norm.weight"], k_norm=norms[f"{attn}.k_norm.weight"]))
    model = ref.LiteSparkQwen(c, layers, np.load(CACHE_DIR / "embedding.int4.npy", allow_pickle=False),
                              np.load(CACHE_DIR / "embedding.scales.npy", allow_pickle=False),
                              norms["model.norm.weight"], SpecKernel())
    assert model.int4_kernel is None and model.attention_kernel is None
    state = model.new_state(len(PROMPT) + DECODE_STEPS)
    fed, logits_all, greedy = [], [], []
    token = None
    for t in PROMPT:
        logits = model.forward_token(t, state)
        fed.append(t)
        logits_all.append(np.array(logits, copy=True))
        token = int(np.asarray(logits).argmax())
        greedy.append(token)
    for _ in range(DECODE_STEPS - 1):
        logits = model.forward_token(token, state)
        fed.append(token)
        logits_all.append(np.array(logits, copy=True))
        token = int(np.asarray(logits).argmax())
        greedy.append(token)

    out = {
        "config_json": np.frombuffer(json.dumps(c, sort_keys=True).encode(), dtype=np.uint8),
        "identity_json": np.frombuffer(json.dumps(identity, sort_keys=True).encode(), dtype=np.uint8),
        "digest": np.frombuffer(digest.encode(), dtype=np.uint8),
        "norm_names": np.array(list(norms), dtype="U64"),
        "tokens": np.array(fed, dtype=np.int32),
        "logits": np.stack(logits_all).astype(np.float32),
        "greedy": np.array(greedy, dtype=np.int32),
        "rope_cos": np.ascontiguousarray(model.rope_cos), "rope_sin": np.ascontiguousarray(model.rope_sin),
    }
    for i, v in enumerate(norms.values()):
        out[f"norm_{i}"] = v
    np.savez_compressed(OUT, **out)
    print(f"wrote {CACHE_DIR} ({len(names)} projections) and {OUT}: tokens {fed} greedy {greedy}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
