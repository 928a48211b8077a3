"""Random-initialised Qwen3-shaped int4 models built directly in HBM.

The benchmark configurations use synthetic weights (there is no checkpoint
here): integers uniform in [-7,7] packed two per byte in the reference
layout (cpu_lightspark.py:139-146 in the reference repository), per-row fp32
scales ~U(0.005, 0.02), norm weights ~U(0.9, 1.1).  A byte is drawn uniformly
from the 225 bytes whose two nibbles are both in [-7,7], which is the same
as drawing each of its two values uniformly from [-7,7].
"""
from __future__ import annotations

import numpy as np
import torch

from .config import shapes
from .lightspark import LiteSparkProjection, LiteSparkQwen, QwenLayer

_VALID = np.array([b for b in range(256) if (b & 0xF) != 8 and (b >> 4) != 8], dtype=np.uint8)


def random_packed(rows: int, width: int, gen: torch.Generator, device) -> torch.Tensor:
    lut = torch.from_numpy(_VALID).to(device)
    out = torch.empty((rows, width // 2), dtype=torch.uint8, device=device)
    step = max(1, (1 << 24) // max(1, width // 2))
    for r0 in range(0, rows, step):
        r1 = min(rows, r0 + step)
        idx = torch.randint(0, len(_VALID), (r1 - r0, width // 2), generator=gen, device=device)
        out[r0:r1] = lut[idx]
    return out


def _uniform(n: int, lo: float, hi: float, gen: torch.Generator, device) -> torch.Tensor:
    return (torch.rand(n, generator=gen, device=device, dtype=torch.float32) * (hi - lo) + lo).contiguous()


def random_model(config: dict, seed: int = 0, device=None) -> LiteSparkQwen:
    device = device or torch.device("cuda", torch.cuda.current_device())
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    h = int(config["hidden_size"])
    d = int(config["head_dim"])
    layers = []
    for _ in range(int(config["num_hidden_layers"])):
        proj = {}
        for name, (rows, width) in shapes(config).items():
            proj[name] = LiteSparkProjection(random_packed(rows, width, gen, device),
                                             _uniform(rows, 0.005, 0.02, gen, device))
        layers.append(QwenLayer(
            qkv=proj["qkv"], o=proj["o"], gate_up=proj["gate_up"], down=proj["down"],
            input_norm=_uniform(h, 0.9, 1.1, gen, device), post_norm=_uniform(h, 0.9, 1.1, gen, device),
            q_norm=_uniform(d, 0.9, 1.1, gen, device), k_norm=_uniform(d, 0.9, 1.1, gen, device)))
    vocab = int(config["vocab_size"])
    embedding = random_packed(vocab, h, gen, device)
    embedding_scales = _uniform(vocab, 0.005, 0.02, gen, device)
    final_norm = _uniform(h, 0.9, 1.1, gen, device)
    return LiteSparkQwen(config, layers, embedding, embedding_scales, final_norm)


def model_from_arrays(config: dict, arrays: dict, device=None) -> LiteSparkQwen:
    """Upload host arrays (keys as in host_arrays) into a device model."""
    device = device or torch.device("cuda", torch.cuda.current_device())

    def t(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(device)

    layers = []
    for i in range(int(config["num_hidden_layers"])):
        proj = {n: LiteSparkProjection(t(arrays[n][i]), t(arrays[n + "_scales"][i]))
                for n in ("qkv", "o", "gate_up", "down")}
        layers.append(QwenLayer(**proj, **{n: t(arrays[n][i]) for n in
                                           ("input_norm", "post_norm", "q_norm", "k_norm")}))
    return LiteSparkQwen(config, layers, t(arrays["embedding"]), t(arrays["embedding_scales"]),
                         t(arrays["final_norm"]))


def host_arrays(model: LiteSparkQwen) -> dict:
    """Host copies of every model buffer, keyed for the CPU oracle."""
    out = {k: [] for k in ("qkv", "qkv_scales", "o", "o_scales", "gate_up", "gate_up_scales",
                           "down", "down_scales", "input_norm", "post_norm", "q_norm", "k_norm")}
    for layer in model.layers:
        for name in ("qkv", "o", "gate_up", "down"):
            p = getattr(layer, name)
            out[name].append(p.weights.cpu().numpy())
            out[name + "_scales"].append(p.scales.cpu().numpy())
        for name in ("input_norm", "post_norm", "q_norm", "k_norm"):
            out[name].append(getattr(layer, name).cpu().numpy())
    out["embedding"] = model.embedding.cpu().numpy()
    out["embedding_scales"] = model.embedding_scales.cpu().numpy()
    out["final_norm"] = model.final_norm.cpu().numpy()
    out["rope_cos"] = model.rope_cos_host
    out["rope_sin"] = model.rope_sin_host
    return out
