"""The reference's on-disk int4 cache, read straight into HBM.

The reference converts a LATTICE checkpoint once into row-quantized int4
projections and keeps them in a cache directory (cpu_lightspark.py:556-686
in the reference repository):

  <directory>/manifest.json                {"identity": {...}, "complete": bool,
                                            "projections": {name: {"weights", "scales"}}}
  <directory>/<slug>.int4.npy              uint8 [rows, width/2], two signed nibbles per byte
  <directory>/<slug>.scales.npy            float32 [rows]
  <directory>/embedding.int4.npy/.scales.npy   the tied embedding / LM head

with slug = the projection name with "." replaced by "_" (:598-600), seven
projections per layer in the order q, k, v, o, gate, up, down (:589-596).
The cache holds no norm weights: those are fp32 tensors of the checkpoint
itself (:663-667, :674), supplied here as a state-dict file (read with
torch.load(weights_only=True), which executes nothing from the file) or as
a mapping of arrays.

Every .npy file is read with numpy.load(allow_pickle=False).  q/k/v and
gate/up are fused by row concatenation as the reference does (:638-662).
The LATTICE-to-int4 conversion itself (:149-201) is not part of this path.
"""
from __future__ import annotations

import hashlib
import json
import os
from pathlib import Path
from typing import Mapping

import numpy as np

CACHE_VERSION = 2
CACHE_FORMAT = "lattice-to-row-int4-litespark"
EMBEDDING_FORMAT = "symmetric-int4-per-row"

_LAYER_PROJECTIONS = (("self_attn", "q_proj"), ("self_attn", "k_proj"), ("self_attn", "v_proj"),
                      ("self_attn", "o_proj"), ("mlp", "gate_proj"), ("mlp", "up_proj"),
                      ("mlp", "down_proj"))


def projection_names(config: dict) -> list[str]:
    """The cached projections in the reference's order (cpu_lightspark.py:584-596)."""
    names = []
    for index in range(int(config["num_hidden_layers"])):
        for block, proj in _LAYER_PROJECTIONS:
            names.append(f"model.layers.{index}.{block}.{proj}")
    return names


def projection_shape(config: dict, name: str) -> tuple[int, int]:
    """(rows, width) of one unfused projection."""
    h = int(config["hidden_size"])
    i = int(config["intermediate_size"])
    d = int(config["head_dim"])
    q = int(config["num_attention_heads"]) * d
    kv = int(config["num_key_value_heads"]) * d
    return {"q_proj": (q, h), "k_proj": (kv, h), "v_proj": (kv, h), "o_proj": (h, q),
            "gate_proj": (i, h), "up_proj": (i, h), "down_proj": (h, i)}[name.rsplit(".", 1)[1]]


def slug(name: str) -> str:
    return name.replace(".", "_")


def identity_digest(identity: dict) -> str:
    """The 16-hex-digit directory name of an identity record
    (cpu_lightspark.py:242)."""
    return hashlib.sha256(json.dumps(identity, sort_keys=True).encode()).hexdigest()[:16]


def cache_identity(model_path) -> tuple[str, dict]:
    """Identity record and directory digest of a checkpoint's cache
    (cpu_lightspark.py:232-243): the cache of model_path lives in
    <cache root>/<digest>."""
    model_path = Path(model_path)
    stat = model_path.stat()
    identity = {
        "version": CACHE_VERSION,
        "source": str(model_path.resolve()),
        "size": stat.st_size,
        "mtime_ns": stat.st_mtime_ns,
        "format": CACHE_FORMAT,
        "embedding": EMBEDDING_FORMAT,
    }
    return identity_digest(identity), identity


def _load_npy(path: Path, dtype, shape: tuple, what: str) -> np.ndarray:
    if not path.exists():
        raise ValueError(f"LiteSpark cache file missing for {what}: {path}")
    array = np.load(path, mmap_mode="r", allow_pickle=False)
    if array.dtype != dtype or tuple(array.shape) != tuple(shape):
        raise ValueError(f"invalid LiteSpark cache shape for {what}")
    return array


def read_manifest(directory, model_path=None, allow_incomplete: bool = False) -> dict:
    """manifest.json of a cache directory, checked as the reference checks it
    (cpu_lightspark.py:574-579): same identity as model_path's when given, a
    supported format, and complete unless allow_incomplete."""
    directory = Path(directory)
    path = directory / "manifest.json"
    if not path.exists():
        raise ValueError(f"no LiteSpark cache manifest in {directory}")
    manifest = json.loads(path.read_text())
    identity = manifest.get("identity", {})
    if model_path is not None and identity != cache_identity(model_path)[1]:
        raise ValueError(f"LiteSpark cache does not match checkpoint: {directory}")
    if identity.get("format") != CACHE_FORMAT or identity.get("embedding") != EMBEDDING_FORMAT:
        raise ValueError(f"unsupported LiteSpark cache format in {directory}")
    if not manifest.get("complete", False) and not allow_incomplete:
        raise ValueError(f"LiteSpark cache is incomplete: {directory}")
    return manifest


def read_cache(directory, config: dict, model_path=None, allow_incomplete: bool = False) -> dict:
    """Host arrays (memory-mapped, read-only) of every cached projection,
    fused as the decode path uses them: keys qkv, o, gate_up, down (+ _scales),
    lists over layers, and embedding / embedding_scales."""
    directory = Path(directory)
    manifest = read_manifest(directory, model_path, allow_incomplete)
    entries = manifest.get("projections", {})
    single = {}
    for name in projection_names(config):
        if name not in entries:
            raise ValueError(f"LiteSpark cache has no entry for {name}")
        files = entries[name]
        rows, width = projection_shape(config, name)
        single[name] = (_load_npy(directory / files["weights"], np.uint8, (rows, width // 2), name),
                        _load_npy(directory / files["scales"], np.float32, (rows,), name))
    out = {k: [] for k in ("qkv", "qkv_scales", "o", "o_scales", "gate_up", "gate_up_scales",
                           "down", "down_scales")}
    for index in range(int(config["num_hidden_layers"])):
        attn = f"model.layers.{index}.self_attn"
        mlp = f"model.layers.{index}.mlp"
        fused = {"qkv": [f"{attn}.q_proj", f"{attn}.k_proj", f"{attn}.v_proj"], "o": [f"{attn}.o_proj"],
                 "gate_up": [f"{mlp}.gate_proj", f"{mlp}.up_proj"], "down": [f"{mlp}.down_proj"]}
        for key, names in fused.items():
            out[key].append(np.concatenate([single[n][0] for n in names], axis=0))
            out[key + "_scales"].append(np.concatenate([single[n][1] for n in names]))
    vocab, hidden = int(config["vocab_size"]), int(config["hidden_size"])
    out["embedding"] = _load_npy(directory / "embedding.int4.npy", np.uint8, (vocab, hidden // 2), "embedding")
    out["embedding_scales"] = _load_npy(directory / "embedding.scales.npy", np.float32, (vocab,), "embedding")
    return out


def norm_keys(config: dict) -> dict:
    """State-dict names of the fp32 norm weights (cpu_lightspark.py:663-667, 674)."""
    keys = {"input_norm": [], "post_norm": [], "q_norm": [], "k_norm": []}
    for index in range(int(config["num_hidden_layers"])):
        prefix = f"model.layers.{index}"
        keys["input_norm"].append(f"{prefix}.input_layernorm.weight")
        keys["post_norm"].append(f"{prefix}.post_attention_layernorm.weight")
        keys["q_norm"].append(f"{prefix}.self_attn.q_norm.weight")
        keys["k_norm"].append(f"{prefix}.self_attn.k_norm.weight")
    keys["final_norm"] = "model.norm.weight"
    return keys


def read_norms(source, config: dict) -> dict:
    """fp32 norm weights from a state-dict file (torch.load with
    weights_only=True) or a mapping of name -> array-like."""
    if isinstance(source, (str, os.PathLike)):
        import torch
        state = torch.load(source, map_location="cpu", weights_only=True, mmap=True)
    elif isinstance(source, Mapping):
        state = source
    else:
        raise TypeError("norm weights come from a state-dict path or a mapping")
    hidden, head_dim = int(config["hidden_size"]), int(config["head_dim"])

    def fetch(key: str, n: int) -> np.ndarray:
        if key not in state:
            raise ValueError(f"norm weight {key} is missing")
        value = state[key]
        array = value.float().numpy() if hasattr(value, "float") else np.asarray(value, dtype=np.float32)
        array = np.array(array, dtype=np.float32, copy=True).reshape(-1)
        if array.shape != (n,):
            raise ValueError(f"norm weight {key} has shape {array.shape}, expected ({n},)")
        return array

    keys = norm_keys(config)
    out = {k: [fetch(name, hidden if k in ("input_norm", "post_norm") else head_dim) for name in keys[k]]
           for k in ("input_norm", "post_norm", "q_norm", "k_norm")}
    out["final_norm"] = fetch(keys["final_norm"], hidden)
    return out


def load_litespark_cache(directory, norms, config: dict | None = None, model_path=None, device=None):
    """A device model (LiteSparkQwen) from the reference's cache directory and
    the checkpoint's norm weights: the int4 bytes are uploaded unchanged."""
    from .config import QWEN3_4B
    from .synthetic import model_from_arrays
    config = dict(config or QWEN3_4B)
    arrays = read_cache(directory, config, model_path)
    arrays.update(read_norms(norms, config))
    return model_from_arrays(config, arrays, device=device)


def write_cache(directory, config: dict, single: Mapping, embedding: np.ndarray, embedding_scales: np.ndarray,
                identity: dict | None = None, complete: bool = True) -> Path:
    """Write a cache in the reference's layout from unfused host arrays
    (single[name] = (uint8 [rows, width/2], float32 [rows]) for every name of
    projection_names(config)); used to check the reader against the format."""
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    manifest = {"identity": identity or {"version": CACHE_VERSION, "source": "", "size": 0, "mtime_ns": 0,
                                         "format": CACHE_FORMAT, "embedding": EMBEDDING_FORMAT},
                "complete": complete, "projections": {}}
    for name in projection_names(config):
        weights, scales = single[name]
        wname, sname = f"{slug(name)}.int4.npy", f"{slug(name)}.scales.npy"
        np.save(directory / wname, np.ascontiguousarray(weights, dtype=np.uint8))
        np.save(directory / sname, np.ascontiguousarray(scales, dtype=np.float32))
        manifest["projections"][name] = {"weights": wname, "scales": sname}
    np.save(directory / "embedding.int4.npy", np.ascontiguousarray(embedding, dtype=np.uint8))
    np.save(directory / "embedding.scales.npy", np.ascontiguousarray(embedding_scales, dtype=np.float32))
    (directory / "manifest.json").write_text(json.dumps(manifest, indent=2, sort_keys=True))
    return directory


def split_fused(config: dict, arrays: Mapping) -> dict:
    """Unfused (name -> (weights, scales)) from fused host arrays (the inverse
    of read_cache's row concatenation)."""
    d = int(config["head_dim"])
    q = int(config["num_attention_heads"]) * d
    kv = int(config["num_key_value_heads"]) * d
    i = int(config["intermediate_size"])
    out = {}
    for index in range(int(config["num_hidden_layers"])):
        attn = f"model.layers.{index}.self_attn"
        mlp = f"model.layers.{index}.mlp"
        w, s = arrays["qkv"][index], arrays["qkv_scales"][index]
        out[f"{attn}.q_proj"] = (w[:q], s[:q])
        out[f"{attn}.k_proj"] = (w[q:q + kv], s[q:q + kv])
        out[f"{attn}.v_proj"] = (w[q + kv:], s[q + kv:])
        out[f"{attn}.o_proj"] = (arrays["o"][index], arrays["o_scales"][index])
        w, s = arrays["gate_up"][index], arrays["gate_up_scales"][index]
        out[f"{mlp}.gate_proj"] = (w[:i], s[:i])
        out[f"{mlp}.up_proj"] = (w[i:], s[i:])
        out[f"{mlp}.down_proj"] = (arrays["down"][index], arrays["down_scales"][index])
    return out
