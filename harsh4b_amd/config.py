"""Model shapes.  QWEN3_4B restates configs/qwen3-4b.json of the reference
repository (the fields the decode path reads)."""

QWEN3_4B = {
    "hidden_size": 2560,
    "intermediate_size": 9728,
    "num_attention_heads": 32,
    "num_key_value_heads": 8,
    "head_dim": 128,
    "num_hidden_layers": 36,
    "vocab_size": 151936,
    "rms_norm_eps": 1e-06,
    "rope_theta": 1000000,
    "max_position_embeddings": 40960,
    "tie_word_embeddings": True,
}


def shapes(config: dict) -> dict:
    """Packed projection shapes (rows, width) of one layer, fused as the
    reference fuses them (cpu_lightspark.py:638-662)."""
    h = int(config["hidden_size"])
    i = int(config["intermediate_size"])
    d = int(config["head_dim"])
    q = int(config["num_attention_heads"]) * d
    kv = int(config["num_key_value_heads"]) * d
    return {"qkv": (q + 2 * kv, h), "o": (h, q), "gate_up": (2 * i, h), "down": (h, i)}


def body_bytes(config: dict) -> int:
    """Packed body-weight bytes read per token (all layers)."""
    per_layer = sum(r * w // 2 for r, w in shapes(config).values())
    return per_layer * int(config["num_hidden_layers"])
