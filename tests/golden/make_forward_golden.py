"""Golden vectors for the decode-step composition (forward_token).

``forward_token`` (cpu_lightspark.py:424-468 in the reference repository)
composes per-op functions that are pinned elsewhere; its composition (the
order of norms, projections, rope, KV write, attention, residuals, SwiGLU and
the LM head) is pinned here by running the reference's own Python
``LiteSparkQwen.forward_token`` on a tiny random model in this container.

The reference's native library is Apple-only and its third-party
``litespark_inference`` kernel object is absent, so:
  * the int4 projections take the reference's non-native branch
    (``kernel.lm_head_int4``, :361-366) and attention takes its numpy
    branch (:408-422);
  * the kernel object is a stand-in whose rmsnorm_into /
    quantize_activation / add_inplace / lm_head_int4 call this repository's
    CPU oracle (the spec those steps follow, pinned by their own tests).
The KV cache is the reference's fp32 QwenDecodeState cache.

Output: tests/golden/forward_tiny.npz (plain arrays: inputs and outputs).
Run:    python tests/golden/make_forward_golden.py [/path/to/reference]
"""
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
OUT = HERE / "forward_tiny.npz"

CONFIG = {
    "hidden_size": 128, "intermediate_size": 256, "num_attention_heads": 2,
    "num_key_value_heads": 1, "head_dim": 128, "num_hidden_layers": 2,
    "vocab_size": 512, "rms_norm_eps": 1e-6, "rope_theta": 1000000,
    "max_position_embeddings": 64,
}
PROMPT = [17, 300, 5, 511, 42]
DECODE_STEPS = 6


def random_int4(rng, rows, width):
    return rng.integers(-7, 8, size=(rows, width), dtype=np.int8)


def main(reference_root: str) -> None:
    sys.path.insert(0, str(REPO))
    sys.path.insert(0, reference_root)
    import oracle  # noqa: E402  (the spec functions of the stand-in kernel)
    from cpu_lightspark import LiteSparkProjection, LiteSparkQwen, QwenLayer, _pack_int4

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
    nq, nkv, d = c["num_attention_heads"], c["num_key_value_heads"], c["head_dim"]
    rng = np.random.default_rng(2024)
    arrays = {k: [] for k in ("qkv", "qkv_scales", "o", "o_scales", "gate_up",
                              "gate_up_scales", "down", "down_scales", "input_norm",
                              "post_norm", "q_norm", "k_norm")}
    layers = []
    for _ in range(c["num_hidden_layers"]):
        shapes = {"qkv": (nq * d + 2 * nkv * d, H), "o": (H, nq * d),
                  "gate_up": (2 * I, H), "down": (H, I)}
        proj = {}
        for name, (rows, width) in shapes.items():
            w = _pack_int4(random_int4(rng, rows, width))
            s = rng.uniform(0.005, 0.02, size=rows).astype(np.float32)
            arrays[name].append(w)
            arrays[name + "_scales"].append(s)
            proj[name] = LiteSparkProjection(w, s)
        norms = {}
        for name, n in (("input_norm", H), ("post_norm", H), ("q_norm", d), ("k_norm", d)):
            g = rng.uniform(0.5, 1.5, size=n).astype(np.float32)
            arrays[name].append(g)
            norms[name] = g
        layers.append(QwenLayer(qkv=proj["qkv"], o=proj["o"], gate_up=proj["gate_up"],
                                down=proj["down"], **norms))
    embedding = _pack_int4(random_int4(rng, c["vocab_size"], H))
    embedding_scales = rng.uniform(0.005, 0.02, size=c["vocab_size"]).astype(np.float32)
    final_norm = rng.uniform(0.5, 1.5, size=H).astype(np.float32)

    model = LiteSparkQwen(c, layers, embedding, embedding_scales, final_norm, SpecKernel())
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
        "tokens": np.array(fed, dtype=np.int32),
        "logits": np.stack(logits_all).astype(np.float32),
        "greedy": np.array(greedy, dtype=np.int32),
        "final_x": np.array(state.x, copy=True),
        "keys": np.array(state.keys, copy=True), "values": np.array(state.values, copy=True),
        "embedding": embedding, "embedding_scales": embedding_scales,
        "final_norm": final_norm,
        "rope_cos": np.ascontiguousarray(model.rope_cos), "rope_sin": np.ascontiguousarray(model.rope_sin),
    }
    for name, items in arrays.items():
        out[name] = np.stack(items)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: tokens {fed} greedy {greedy}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
