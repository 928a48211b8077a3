"""ctypes bindings of the CPU oracle (``liborhq.so``, built from hq_oracle.c).

TEST INFRASTRUCTURE ONLY.  The oracle is the checker the HIP product path is
compared against.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` import this module; ``harsh4b_amd``
never does.  Each wrapper names the reference lines its C function restates
(paths relative to the reference repository).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liborhq.so"

_c_i8p = ctypes.POINTER(ctypes.c_int8)
_c_u8p = ctypes.POINTER(ctypes.c_uint8)
_c_u16p = ctypes.POINTER(ctypes.c_uint16)
_c_i32p = ctypes.POINTER(ctypes.c_int32)
_c_f32p = ctypes.POINTER(ctypes.c_float)


def build(force: bool = False) -> Path:
    """Compile liborhq.so with oracle/Makefile (gcc, OpenMP)."""
    if force and LIB_PATH.exists():
        LIB_PATH.unlink()
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


_LIB = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            build()
        _LIB = ctypes.CDLL(str(LIB_PATH))
        _declare(_LIB)
    return _LIB


class OrLayer(ctypes.Structure):
    _fields_ = [
        ("qkv", _c_u8p), ("qkv_scales", _c_f32p),
        ("o", _c_u8p), ("o_scales", _c_f32p),
        ("gate_up", _c_u8p), ("gate_up_scales", _c_f32p),
        ("down", _c_u8p), ("down_scales", _c_f32p),
        ("input_norm", _c_f32p), ("post_norm", _c_f32p),
        ("q_norm", _c_f32p), ("k_norm", _c_f32p),
    ]


class OrModel(ctypes.Structure):
    _fields_ = [
        ("layers", ctypes.c_int32), ("hidden", ctypes.c_int32),
        ("intermediate", ctypes.c_int32), ("heads", ctypes.c_int32),
        ("kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("vocab", ctypes.c_int32), ("rope_positions", ctypes.c_int32),
        ("eps", ctypes.c_float), ("chunk", ctypes.c_int32),
        ("layer", ctypes.POINTER(OrLayer)),
        ("embedding", _c_u8p), ("embedding_scales", _c_f32p),
        ("final_norm", _c_f32p), ("rope_cos", _c_f32p), ("rope_sin", _c_f32p),
    ]


class OrState(ctypes.Structure):
    _fields_ = [
        ("capacity", ctypes.c_int32), ("position", ctypes.c_int32),
        ("kv_f32", ctypes.c_int32), ("pad", ctypes.c_int32),
        ("keys", ctypes.c_void_p), ("values", ctypes.c_void_p),
        ("x", _c_f32p), ("logits", _c_f32p), ("trace", _c_f32p),
    ]


def _declare(L: ctypes.CDLL) -> None:
    vp = ctypes.c_void_p
    L.or_expf.argtypes = [ctypes.c_float]
    L.or_expf.restype = ctypes.c_float
    L.or_f32_to_f16_array.argtypes = [vp, vp, ctypes.c_int64]
    L.or_f16_to_f32_array.argtypes = [vp, vp, ctypes.c_int64]
    L.or_pack_int4.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp]
    L.or_pack_int4.restype = ctypes.c_int
    L.or_unpack_int4.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp]
    L.or_unpack_int4.restype = ctypes.c_int
    L.or_quantize_activation.argtypes = [vp, ctypes.c_int, vp]
    L.or_quantize_activation.restype = ctypes.c_float
    L.or_rmsnorm.argtypes = [vp, vp, vp, ctypes.c_int, ctypes.c_float]
    L.or_head_norm.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_float]
    L.or_rope.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp, vp]
    L.or_int4_i8_gemv.argtypes = [vp, vp, vp, ctypes.c_float, vp, ctypes.c_int, ctypes.c_int]
    L.or_int4_i8_gemv_acc.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, vp]
    L.or_set_simd.argtypes = [ctypes.c_int]
    L.or_set_simd.restype = None
    L.or_simd_active.argtypes = []
    L.or_set_threads.argtypes = [ctypes.c_int]
    L.or_set_threads.restype = None
    L.or_max_threads.argtypes = []
    L.or_int4_i8_gemm_acc.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp]
    L.or_quant_int4_gemv.argtypes = [vp, vp, vp, vp, ctypes.c_int, ctypes.c_int, vp, vp]
    L.or_quant_int4_gemv.restype = ctypes.c_float
    L.or_gqa_decode_ref.argtypes = [vp] * 5 + [ctypes.c_int] * 5
    L.or_gqa_decode_split.argtypes = [vp] * 4 + [ctypes.c_int] * 4 + [ctypes.c_int64, ctypes.c_int]
    L.or_gqa_decode_split_f32.argtypes = [vp] * 4 + [ctypes.c_int] * 4 + [ctypes.c_int64, ctypes.c_int]
    L.or_swiglu.argtypes = [vp, vp, vp, ctypes.c_int]
    L.or_argmax.argtypes = [vp, ctypes.c_int64]
    L.or_pairwise_sum_f32.argtypes = [vp, ctypes.c_int]
    L.or_pairwise_sum_f32.restype = ctypes.c_float
    L.or_sample_token.argtypes = [vp, ctypes.c_int64, vp, ctypes.c_int, ctypes.c_float, ctypes.c_float,
                                  ctypes.c_int, ctypes.c_float, ctypes.c_double, vp, vp]
    L.or_sample_token.restype = ctypes.c_int64
    L.or_argmax.restype = ctypes.c_int64
    L.or_embedding.argtypes = [ctypes.POINTER(OrModel), ctypes.c_int, vp]
    L.or_forward_token.argtypes = [ctypes.POINTER(OrModel), ctypes.POINTER(OrState), ctypes.c_int]
    L.or_forward_token.restype = ctypes.c_int


def _p(a: np.ndarray):
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("oracle arrays must be C-contiguous")
    return a.ctypes.data


# ---------------------------------------------------------------- scalar spec
def expf(x) -> np.ndarray:
    """Spec exp (Cody-Waite + degree-7 Taylor); elementwise."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    f = lib().or_expf
    return np.array([f(float(v)) for v in x.reshape(-1)], dtype=np.float32).reshape(x.shape)


def f32_to_f16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().or_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().or_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


# ---------------------------------------------------------------- packing
def pack_int4(weights: np.ndarray) -> np.ndarray:
    """cpu_lightspark.py:139-146."""
    w = np.ascontiguousarray(weights, dtype=np.int8)
    rows, width = w.shape
    out = np.empty((rows, width // 2), dtype=np.uint8)
    rc = lib().or_pack_int4(_p(w), rows, width, _p(out))
    if rc == -2:
        raise ValueError("int4 matrix must be int8 with even width")
    if rc == -1:
        raise ValueError("int4 values must be in [-7,+7]")
    return out


def unpack_int4(packed: np.ndarray, width: int) -> np.ndarray:
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty((p.shape[0], width), dtype=np.int8)
    if lib().or_unpack_int4(_p(p), p.shape[0], width, _p(out)) != 0:
        raise ValueError("odd width")
    return out


# ---------------------------------------------------------------- quantization, norms
def quantize_activation(x: np.ndarray):
    """Returns (int8 vector, act_scale)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(x.shape, dtype=np.int8)
    s = lib().or_quantize_activation(_p(x), x.size, _p(q))
    return q, np.float32(s)


def rmsnorm(x: np.ndarray, gamma: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = np.ascontiguousarray(gamma, dtype=np.float32)
    y = np.empty_like(x)
    lib().or_rmsnorm(_p(x), _p(g), _p(y), x.size, eps)
    return y


def head_norm(x: np.ndarray, gamma: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    g = np.ascontiguousarray(gamma, dtype=np.float32)
    lib().or_head_norm(_p(y), _p(g), y.shape[0], y.shape[1], eps)
    return y


def rope(x: np.ndarray, cos_row: np.ndarray, sin_row: np.ndarray) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    c = np.ascontiguousarray(cos_row, dtype=np.float32)
    s = np.ascontiguousarray(sin_row, dtype=np.float32)
    lib().or_rope(_p(y), y.shape[0], y.shape[1], _p(c), _p(s))
    return y


# ---------------------------------------------------------------- int4 GEMV
def int4_i8_gemv(x, weights, scales, activation_scale, rows, width) -> np.ndarray:
    """litespark_int4.cpp:78-108 signature."""
    x = np.ascontiguousarray(x, dtype=np.int8)
    w = np.ascontiguousarray(weights, dtype=np.uint8)
    s = np.ascontiguousarray(scales, dtype=np.float32)
    out = np.empty(rows, dtype=np.float32)
    lib().or_int4_i8_gemv(_p(x), _p(w), _p(s), float(activation_scale), _p(out), rows, width)
    return out


def int4_i8_gemv_acc(x, weights, rows, width) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.int8)
    w = np.ascontiguousarray(weights, dtype=np.uint8)
    acc = np.empty(rows, dtype=np.int32)
    lib().or_int4_i8_gemv_acc(_p(x), _p(w), rows, width, _p(acc))
    return acc


def int4_i8_gemm_acc(x, weights, rows, width) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.int8)
    w = np.ascontiguousarray(weights, dtype=np.uint8)
    m = x.shape[0]
    acc = np.empty((m, rows), dtype=np.int32)
    lib().or_int4_i8_gemm_acc(_p(x), _p(w), m, rows, width, _p(acc))
    return acc


def quant_int4_gemv(x, weights, scales):
    """Fused quantization + GEMV.  Returns (out fp32, q int8, act_scale, acc int32)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(weights, dtype=np.uint8)
    s = np.ascontiguousarray(scales, dtype=np.float32)
    rows, width = w.shape[0], x.size
    out = np.empty(rows, dtype=np.float32)
    q = np.empty(width, dtype=np.int8)
    acc = np.empty(rows, dtype=np.int32)
    act = lib().or_quant_int4_gemv(_p(x), _p(w), _p(s), _p(out), rows, width, _p(q), _p(acc))
    return out, q, np.float32(act), acc


# ---------------------------------------------------------------- GQA decode attention
def gqa_decode_ref(query, keys, values, context, kv_heads, groups, head_dim, capacity):
    """litespark_int4.cpp:160-259 with fp32 keys/values [capacity, kv, d]."""
    q = np.ascontiguousarray(query, dtype=np.float32)
    k = np.ascontiguousarray(keys, dtype=np.float32)
    v = np.ascontiguousarray(values, dtype=np.float32)
    scores = np.zeros((kv_heads * groups, capacity), dtype=np.float32)
    out = np.empty((kv_heads * groups, head_dim), dtype=np.float32)
    lib().or_gqa_decode_ref(_p(q), _p(k), _p(v), _p(scores), _p(out), context,
                            kv_heads, groups, head_dim, capacity)
    return out, scores


def gqa_decode_split(query, keys16, values16, context, kv_heads, groups, head_dim, chunk=64):
    """Spec-order split attention over fp16 keys/values [time, kv, d] (uint16 bits)."""
    q = np.ascontiguousarray(query, dtype=np.float32)
    k = np.ascontiguousarray(keys16, dtype=np.uint16)
    v = np.ascontiguousarray(values16, dtype=np.uint16)
    out = np.empty((kv_heads * groups, head_dim), dtype=np.float32)
    lib().or_gqa_decode_split(_p(q), _p(k), _p(v), _p(out), context, kv_heads, groups,
                              head_dim, kv_heads * head_dim, chunk)
    return out


def gqa_decode_split_f32(query, keys, values, context, kv_heads, groups, head_dim, chunk=64):
    """Spec-order split attention over fp32 keys/values [time, kv, d]."""
    q = np.ascontiguousarray(query, dtype=np.float32)
    k = np.ascontiguousarray(keys, dtype=np.float32)
    v = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty((kv_heads * groups, head_dim), dtype=np.float32)
    lib().or_gqa_decode_split_f32(_p(q), _p(k), _p(v), _p(out), context, kv_heads, groups,
                                  head_dim, kv_heads * head_dim, chunk)
    return out


# ---------------------------------------------------------------- SwiGLU, argmax, sampler
def swiglu(gate, up) -> np.ndarray:
    g = np.ascontiguousarray(gate, dtype=np.float32)
    u = np.ascontiguousarray(up, dtype=np.float32)
    out = np.empty_like(g)
    lib().or_swiglu(_p(g), _p(u), _p(out), g.size)
    return out


def argmax(x) -> int:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return int(lib().or_argmax(_p(x), x.size))


def pairwise_sum_f32(a) -> np.float32:
    a = np.ascontiguousarray(a, dtype=np.float32)
    return np.float32(lib().or_pairwise_sum_f32(_p(a), a.size))


def sample_token(logits, generated, repetition_penalty, temperature, top_k, top_p, u):
    """The reference's stochastic sampler (cpu_lightspark.py:706-726) with the
    uniform draw u given: returns (token, ids [k], probabilities [k])."""
    x = np.ascontiguousarray(logits, dtype=np.float32).reshape(-1)
    g = np.ascontiguousarray(generated, dtype=np.int32).reshape(-1)
    k = max(1, min(int(top_k), x.size))
    ids = np.empty(k, np.int32)
    probs = np.empty(k, np.float32)
    tok = lib().or_sample_token(_p(x), x.size, _p(g) if g.size else None, g.size, float(repetition_penalty),
                                float(temperature), int(top_k), float(top_p), float(u), _p(ids), _p(probs))
    return int(tok), ids, probs


# ---------------------------------------------------------------- decode step
class OracleModel:
    """Host copy of a model in the oracle's struct form.

    ``arrays`` holds numpy arrays keyed like harsh4b_amd.synthetic's host
    export: per-layer lists ``qkv, qkv_scales, o, ..., k_norm`` and the
    globals ``embedding, embedding_scales, final_norm, rope_cos, rope_sin``.
    """

    def __init__(self, config: dict, arrays: dict, chunk: int = 64):
        self.config = config
        self.arrays = arrays  # keeps every buffer alive
        n_layers = int(config["num_hidden_layers"])
        self._layers = (OrLayer * n_layers)()
        for i in range(n_layers):
            lay = self._layers[i]
            for name in ("qkv", "o", "gate_up", "down"):
                setattr(lay, name, _ptr(arrays[name][i], _c_u8p))
                setattr(lay, name + "_scales", _ptr(arrays[name + "_scales"][i], _c_f32p))
            for name in ("input_norm", "post_norm", "q_norm", "k_norm"):
                setattr(lay, name, _ptr(arrays[name][i], _c_f32p))
        m = OrModel()
        m.layers = n_layers
        m.hidden = int(config["hidden_size"])
        m.intermediate = int(config["intermediate_size"])
        m.heads = int(config["num_attention_heads"])
        m.kv_heads = int(config["num_key_value_heads"])
        m.head_dim = int(config["head_dim"])
        m.vocab = int(config["vocab_size"])
        m.rope_positions = int(arrays["rope_cos"].shape[0])
        m.eps = float(config["rms_norm_eps"])
        m.chunk = chunk
        m.layer = self._layers
        m.embedding = _ptr(arrays["embedding"], _c_u8p)
        m.embedding_scales = _ptr(arrays["embedding_scales"], _c_f32p)
        m.final_norm = _ptr(arrays["final_norm"], _c_f32p)
        m.rope_cos = _ptr(arrays["rope_cos"], _c_f32p)
        m.rope_sin = _ptr(arrays["rope_sin"], _c_f32p)
        self.struct = m

    def new_state(self, capacity: int, trace: bool = False, kv_f32: bool = False) -> "OracleState":
        return OracleState(self, capacity, trace, kv_f32)

    def forward_token(self, token: int, state: "OracleState") -> int:
        rc = lib().or_forward_token(ctypes.byref(self.struct), ctypes.byref(state.struct), int(token))
        if rc == -1:
            raise ValueError("decode state capacity exhausted")
        if rc == -2:
            raise ValueError(f"token ID {token} is outside the vocabulary")
        return rc

    def embedding(self, token: int) -> np.ndarray:
        out = np.empty(int(self.config["hidden_size"]), dtype=np.float32)
        lib().or_embedding(ctypes.byref(self.struct), int(token), _p(out))
        return out


class OracleState:
    """KV cache [layers, capacity, kv_heads, head_dim]: fp16 bits (uint16) by
    default, or fp32 as in the reference's QwenDecodeState (kv_f32=True)."""

    def __init__(self, model: OracleModel, capacity: int, trace: bool = False,
                 kv_f32: bool = False):
        c = model.config
        layers = int(c["num_hidden_layers"])
        kv, d = int(c["num_key_value_heads"]), int(c["head_dim"])
        dtype = np.float32 if kv_f32 else np.uint16
        self.keys = np.zeros((layers, capacity, kv, d), dtype=dtype)
        self.values = np.zeros_like(self.keys)
        self.x = np.zeros(int(c["hidden_size"]), dtype=np.float32)
        self.logits = np.zeros(int(c["vocab_size"]), dtype=np.float32)
        self.trace = np.zeros((layers, int(c["hidden_size"])), dtype=np.float32) if trace else None
        s = OrState()
        s.capacity = capacity
        s.position = 0
        s.kv_f32 = 1 if kv_f32 else 0
        s.keys = self.keys.ctypes.data
        s.values = self.values.ctypes.data
        s.x = _ptr(self.x, _c_f32p)
        s.logits = _ptr(self.logits, _c_f32p)
        s.trace = _ptr(self.trace, _c_f32p) if trace else ctypes.cast(None, _c_f32p)
        self.struct = s

    @property
    def position(self) -> int:
        return int(self.struct.position)

    @position.setter
    def position(self, value: int) -> None:
        self.struct.position = int(value)


def _ptr(a: np.ndarray, ctype):
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("oracle arrays must be C-contiguous")
    return ctypes.cast(a.ctypes.data, ctype)


def threads() -> int:
    """OpenMP threads the oracle's GEMVs run on."""
    return int(lib().or_max_threads())


def set_threads(n: int) -> None:
    lib().or_set_threads(int(n))


def set_simd(on: bool) -> None:
    """Use the AVX-512 VNNI GEMV path where the CPU has it (default), or
    force the scalar loop (the same integers)."""
    lib().or_set_simd(int(bool(on)))


def simd_active() -> bool:
    return bool(lib().or_simd_active())
