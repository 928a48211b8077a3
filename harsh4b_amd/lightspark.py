"""MI355X decode runtime with the call surface of cpu_lightspark.py.

Mirrors the reference's decode path (cpu_lightspark.py in the reference
repository) on one gfx950 GPU:

  reference (CPU, numpy + ctypes)          here (HIP via libhq.so + torch plumbing)
  _pack_int4                 :139-146      pack_int4 (same layout, same errors)
  LiteSparkProjection        :246-260      LiteSparkProjection (device buffers)
  combine                    :638-645      combine
  QwenLayer                  :263-272      QwenLayer
  QwenDecodeState            :275-309      QwenDecodeState (fp16 KV cache on HBM)
  LiteSparkQwen.__init__     :315-336      LiteSparkQwen (RoPE tables as :329-336)
  new_state / forward_token  :338, :424    new_state / forward_token
  _projection                :351-371      _projection (hq_int4_i8_gemv)
  _attention                 :389-422      _attention (hq_gqa_decode)
  sample_logits              :700-726      sample_logits (hq_argmax / hq_sample_token)

All arithmetic runs in libhq.so; torch only allocates device memory and
provides the stream.  There is no CPU fallback: a missing library or GPU is
an error.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _native
from ._native import HqLayer, HqModel, HqState, check

DEFAULT_GEMV_KERNEL = "hip-gfx950"


# --------------------------------------------------------------------------- packing
def pack_int4(weights: np.ndarray) -> np.ndarray:
    """Pack signed [-7,+7] values as low/high nibbles (cpu_lightspark.py:139-146)."""
    if weights.dtype != np.int8 or weights.ndim != 2 or weights.shape[1] % 2:
        raise ValueError("int4 matrix must be int8 with even width")
    if np.any(weights < -7) or np.any(weights > 7):
        raise ValueError("int4 values must be in [-7,+7]")
    return ((weights[:, 0::2].view(np.uint8) & 15)
            | ((weights[:, 1::2].view(np.uint8) & 15) << 4))


def _device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("harsh4b_amd needs a ROCm GPU (gfx950); none is visible")
    return torch.device("cuda", torch.cuda.current_device())


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream_handle(stream: torch.cuda.Stream | None) -> int | None:
    """The HIP stream of `stream`, or torch's current stream when None (so
    the op is ordered with the caller's other torch work)."""
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


# --------------------------------------------------------------------------- projections
@dataclass(frozen=True)
class LiteSparkProjection:
    """One row-scaled int4 matrix held on the device (cpu_lightspark.py:246-260)."""

    weights: torch.Tensor          # uint8 [rows, width/2]
    scales: torch.Tensor           # float32 [rows]
    layout: str = "int4"

    def __post_init__(self):
        if self.layout != "int4":
            raise ValueError("only the packed int4 layout is supported on the GPU")
        w, s = self.weights, self.scales
        if w.dtype != torch.uint8 or w.ndim != 2 or not w.is_cuda or not w.is_contiguous():
            raise ValueError("weights must be a contiguous uint8 [rows, width/2] device tensor")
        if s.dtype != torch.float32 or s.shape != (w.shape[0],) or not s.is_cuda:
            raise ValueError("scales must be a float32 [rows] device tensor")

    @property
    def input_size(self) -> int:
        return self.weights.shape[1] * 2

    @property
    def output_size(self) -> int:
        return self.weights.shape[0]


def combine(*projections: LiteSparkProjection) -> LiteSparkProjection:
    """Concatenate rows of projections sharing an input (cpu_lightspark.py:638-645)."""
    if len({item.input_size for item in projections}) != 1:
        raise ValueError("cannot fuse LiteSpark projections with different input widths")
    return LiteSparkProjection(
        torch.cat([item.weights for item in projections], dim=0).contiguous(),
        torch.cat([item.scales for item in projections]).contiguous(),
        projections[0].layout,
    )


@dataclass(frozen=True)
class QwenLayer:
    qkv: LiteSparkProjection
    o: LiteSparkProjection
    gate_up: LiteSparkProjection
    down: LiteSparkProjection
    input_norm: torch.Tensor
    post_norm: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor


def rope_tables(config: dict) -> tuple[np.ndarray, np.ndarray]:
    """cos/sin [max_position_embeddings, head_dim/2] exactly as cpu_lightspark.py:329-336."""
    head_dim = int(config["head_dim"])
    positions = np.arange(int(config["max_position_embeddings"]), dtype=np.float32)[:, None]
    inv_freq = np.float32(1.0) / np.float32(config["rope_theta"]) ** (
        np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim)
    )
    angles = positions * inv_freq[None, :]
    return np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)


# --------------------------------------------------------------------------- decode state
class QwenDecodeState:
    """Caller-owned device state for one sequence (cpu_lightspark.py:275-309).

    The KV cache is fp16 [layers, capacity, kv_heads, head_dim] (the reference
    keeps fp32; the benchmark configurations specify fp16).  Position and the
    current token also live on the device so a captured HIP graph of a step is
    valid at every position; ``position`` here is the host's mirror of it.

    ``stream`` is the model's stream, shared by every state of the model: a
    step's persistent layer kernel needs every CU of the GPU at once, so the
    steps of different sequences run one after another, never side by side
    (concurrent launches would starve each other's waits, HQ_STEP_SYNC).
    """

    def __init__(self, model: "LiteSparkQwen", capacity: int):
        if capacity < 1:
            raise ValueError("decode capacity must be positive")
        c = model.config
        dev = model.device
        layers = int(c["num_hidden_layers"])
        hidden = int(c["hidden_size"])
        intermediate = int(c["intermediate_size"])
        heads = int(c["num_attention_heads"])
        kv_heads = int(c["num_key_value_heads"])
        head_dim = int(c["head_dim"])
        if capacity > model.rope_positions:
            raise ValueError("decode capacity exceeds max_position_embeddings")
        self.model = model
        self.capacity = capacity
        self.position = 0
        f32 = dict(dtype=torch.float32, device=dev)
        self.keys = torch.zeros((layers, capacity, kv_heads, head_dim), dtype=torch.float16, device=dev)
        self.values = torch.zeros_like(self.keys)
        self.device_position = torch.zeros(1, dtype=torch.int32, device=dev)
        self.token = torch.zeros(1, dtype=torch.int32, device=dev)
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)
        self.x = torch.zeros(hidden, **f32)
        q_size, kv_size = heads * head_dim, kv_heads * head_dim
        self.qkv = torch.zeros(q_size + 2 * kv_size, **f32)
        self.q = self.qkv[:q_size].view(heads, head_dim)
        self.k = self.qkv[q_size:q_size + kv_size].view(kv_heads, head_dim)
        self.v = self.qkv[q_size + kv_size:].view(kv_heads, head_dim)
        self.attended = torch.zeros(q_size, **f32)
        self.activated = torch.zeros(intermediate, **f32)
        self.logits = torch.zeros(int(c["vocab_size"]), **f32)
        nbytes = _native.lib().hq_step_workspace_bytes(ctypes.byref(model.struct), capacity)
        if nbytes == 0:
            raise ValueError("model shape is not supported by the decode step")
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        self.stream = model.stream
        self.stream.wait_stream(torch.cuda.current_stream(dev))
        s = HqState()
        s.capacity = capacity
        s.keys, s.values = self.keys.data_ptr(), self.values.data_ptr()
        s.position, s.token, s.status = (self.device_position.data_ptr(), self.token.data_ptr(),
                                         self.status.data_ptr())
        s.x, s.qkv, s.attended = self.x.data_ptr(), self.qkv.data_ptr(), self.attended.data_ptr()
        s.activated, s.logits = self.activated.data_ptr(), self.logits.data_ptr()
        s.workspace = self.workspace.data_ptr()
        self.struct = s
        self._graphs = {}          # steps -> captured graph of that many greedy steps
        self._prefill_ws = None

    def synchronize(self) -> None:
        self.stream.synchronize()

    def check_status(self) -> None:
        self.synchronize()
        code = int(self.status.item())
        if code & _native.HQ_STEP_BAD_TOKEN:
            raise ValueError("a token ID outside the vocabulary reached the device")
        if code & _native.HQ_STEP_FULL:
            raise ValueError("decode state capacity exhausted")
        if code & _native.HQ_STEP_SYNC:
            raise RuntimeError("a phase wait of the persistent layer kernel gave up")

    def close(self) -> None:
        for handle in self._graphs.values():
            _native.lib().hq_graph_destroy(handle)
        self._graphs = {}

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# --------------------------------------------------------------------------- model
class LiteSparkQwen:
    """Qwen3 decode runtime on one MI355X (cpu_lightspark.py:312-468)."""

    def __init__(self, config: dict, layers: list[QwenLayer], embedding: torch.Tensor,
                 embedding_scales: torch.Tensor, final_norm: torch.Tensor,
                 gemv_kernel: str = DEFAULT_GEMV_KERNEL):
        self.device = _device()
        _native.lib()
        self.config = config
        self.layers = layers
        self.embedding = embedding
        self.embedding_scales = embedding_scales
        self.lm_head = LiteSparkProjection(embedding, embedding_scales)
        self.final_norm = final_norm
        self.gemv_kernel = gemv_kernel
        cos, sin = rope_tables(config)
        self.rope_cos_host, self.rope_sin_host = cos, sin
        self.rope_cos = torch.from_numpy(cos).to(self.device)
        self.rope_sin = torch.from_numpy(sin).to(self.device)
        self.rope_positions = cos.shape[0]
        n = int(config["num_hidden_layers"])
        if len(layers) != n:
            raise ValueError(f"expected {n} layers, found {len(layers)}")
        self._layer_structs = (HqLayer * n)()
        for i, layer in enumerate(layers):
            ls = self._layer_structs[i]
            for name in ("qkv", "o", "gate_up", "down"):
                proj = getattr(layer, name)
                setattr(ls, name, proj.weights.data_ptr())
                setattr(ls, name + "_scales", proj.scales.data_ptr())
            for name in ("input_norm", "post_norm", "q_norm", "k_norm"):
                setattr(ls, name, getattr(layer, name).data_ptr())
        m = HqModel()
        m.layers = n
        m.hidden = int(config["hidden_size"])
        m.intermediate = int(config["intermediate_size"])
        m.heads = int(config["num_attention_heads"])
        m.kv_heads = int(config["num_key_value_heads"])
        m.head_dim = int(config["head_dim"])
        m.vocab = int(config["vocab_size"])
        m.rope_positions = self.rope_positions
        m.eps = float(config["rms_norm_eps"])
        m.layer = self._layer_structs
        m.embedding = embedding.data_ptr()
        m.embedding_scales = embedding_scales.data_ptr()
        m.final_norm = final_norm.data_ptr()
        m.rope_cos = self.rope_cos.data_ptr()
        m.rope_sin = self.rope_sin.data_ptr()
        # device copy of the layer table: lets a step run its decoder layers
        # as one persistent kernel
        table = bytes(self._layer_structs)
        self._layer_table = torch.frombuffer(bytearray(table), dtype=torch.uint8).to(self.device)
        m.device_layer = self._layer_table.data_ptr()
        m.flags = 0
        self.struct = m
        self._batch_workspaces: dict[int, torch.Tensor] = {}
        self._batch_graph = None   # (key, graph, states) of the last captured batched step
        # every decode state of the model enqueues on this one stream (see
        # QwenDecodeState), and so does the batched step
        self.stream = torch.cuda.Stream(device=self.device)

    @property
    def layer_kernel_blocks(self) -> int:
        """Blocks of the persistent layer kernel a step launches (0: the
        step runs five kernels per decoder layer)."""
        return int(_native.lib().hq_step_layer_blocks(ctypes.byref(self.struct)))

    @property
    def per_layer_kernels(self) -> bool:
        """True when steps run five kernels per decoder layer instead of the
        persistent layer kernel (same results)."""
        return bool(self.struct.flags & _native.HQ_MODEL_PER_LAYER_KERNELS)

    @per_layer_kernels.setter
    def per_layer_kernels(self, value: bool) -> None:
        if value:
            self.struct.flags |= _native.HQ_MODEL_PER_LAYER_KERNELS
        else:
            self.struct.flags &= ~_native.HQ_MODEL_PER_LAYER_KERNELS

    def new_state(self, capacity: int) -> QwenDecodeState:
        return QwenDecodeState(self, capacity)

    # -- one step -------------------------------------------------------------
    def _check_token(self, token_id: int, state: QwenDecodeState) -> None:
        if state.position >= state.capacity:
            raise ValueError("decode state capacity exhausted")
        if token_id < 0 or token_id >= int(self.config["vocab_size"]):
            raise ValueError(f"token ID {token_id} is outside the vocabulary")

    def forward_token(self, token_id: int, state: QwenDecodeState) -> torch.Tensor:
        """Consume one token and return its next-token logits (device tensor).

        The step is enqueued on ``state.stream``; the greedy (argmax) token
        of the logits is written to ``state.token`` by the same step.  The
        caller's current stream waits for the step, so work it enqueues
        there (sample_logits, a copy) reads the finished logits.
        """
        self._check_token(token_id, state)
        with torch.cuda.stream(state.stream):
            state.token.fill_(int(token_id))
        check(_native.lib().hq_decode_step(ctypes.byref(self.struct), ctypes.byref(state.struct),
                                           state.stream.cuda_stream), "hq_decode_step")
        state.position += 1
        torch.cuda.current_stream(self.device).wait_stream(state.stream)
        return state.logits

    def prefill(self, token_ids, state: QwenDecodeState) -> torch.Tensor:
        """Consume a prompt and return the logits after its last token, as a
        loop of forward_token over it would (the reference's prompt loop,
        cpu_lightspark.py:809-810, inference_runtime.py:177-181), with the
        same bits: every token but the last goes through hq_prefill (layer by
        layer for up to 128 tokens at once, the projections as int8 MFMA
        GEMMs), the last through the decode step, which computes the logits
        and the greedy token."""
        ids = np.asarray(list(token_ids), dtype=np.int64).reshape(-1)
        if ids.size == 0:
            raise ValueError("prefill needs at least one token")
        vocab = int(self.config["vocab_size"])
        if ids.min() < 0 or ids.max() >= vocab:
            raise ValueError("a prompt token ID is outside the vocabulary")
        if state.position + ids.size > state.capacity:
            raise ValueError("decode state capacity exhausted")
        head = ids[:-1]
        if head.size:
            lib = _native.lib()
            if state._prefill_ws is None:
                nbytes = lib.hq_prefill_workspace_bytes(ctypes.byref(self.struct), state.capacity)
                if nbytes == 0:
                    raise ValueError("model shape is not supported by the batched prefill")
                state._prefill_ws = torch.zeros(nbytes, dtype=torch.uint8, device=self.device)
            state.stream.wait_stream(torch.cuda.current_stream(self.device))   # the workspace's zero fill
            with torch.cuda.stream(state.stream):
                dev_ids = torch.from_numpy(head.astype(np.int32)).to(self.device)
            check(lib.hq_prefill(ctypes.byref(self.struct), ctypes.byref(state.struct), dev_ids.data_ptr(),
                                 int(head.size), int(state.position), state._prefill_ws.data_ptr(),
                                 state.stream.cuda_stream), "hq_prefill")
            dev_ids.record_stream(state.stream)
            state.position += int(head.size)
        return self.forward_token(int(ids[-1]), state)

    def greedy_token(self, state: QwenDecodeState) -> int:
        state.synchronize()
        return int(state.token.item())

    GRAPH_STEPS = (64, 8, 1)   # greedy steps per captured graph, largest first

    def decode_greedy(self, state: QwenDecodeState, steps: int, use_graph: bool = True,
                      check_status: bool = True) -> None:
        """Run `steps` greedy steps feeding each argmax token back on the device
        (the token already in ``state.token`` is consumed first).

        With `check_status` (the default) the call waits for the steps and
        raises if the device status word reports a bad token, an exhausted
        cache or a persistent-kernel wait that gave up; a caller that times
        the steps passes False and calls ``state.check_status()`` itself."""
        if state.position + steps > state.capacity:
            raise ValueError("decode state capacity exhausted")
        lib = _native.lib()
        if use_graph:
            def graph(n):
                if n not in state._graphs:
                    handle = ctypes.c_void_p()
                    check(lib.hq_graph_capture(ctypes.byref(self.struct), ctypes.byref(state.struct), n,
                                               state.stream.cuda_stream, ctypes.byref(handle)),
                          "hq_graph_capture")
                    state._graphs[n] = handle.value
                return state._graphs[n]
            # up to GRAPH_STEPS[0] steps per graph launch: the GPU idles
            # between consecutive graph launches (about 140 us at batch 1)
            left = steps
            for n in self.GRAPH_STEPS:
                while left >= n:
                    check(lib.hq_graph_launch(graph(n), state.stream.cuda_stream), "hq_graph_launch")
                    left -= n
        else:
            for _ in range(steps):
                check(lib.hq_decode_step(ctypes.byref(self.struct), ctypes.byref(state.struct),
                                         state.stream.cuda_stream), "hq_decode_step")
        state.position += steps
        if check_status:
            state.check_status()

    # -- batched decode (M independent sequences) -------------------------------
    MAX_BATCH = 32

    def _batch_setup(self, states):
        m = len(states)
        if not 1 <= m <= self.MAX_BATCH:
            raise ValueError(f"a batched step takes 1 to {self.MAX_BATCH} decode states")
        if len({id(st) for st in states}) != m:
            raise ValueError("a decode state appears twice in the batch")
        for st in states:
            if st.model is not self:
                raise ValueError("a decode state belongs to another model")
        cap = max(st.capacity for st in states)
        ws = self._batch_workspaces.get(cap)
        if ws is None:
            nbytes = _native.lib().hq_decode_batch_workspace_bytes(ctypes.byref(self.struct), cap)
            if nbytes == 0:
                raise ValueError("model shape is not supported by the batched decode step")
            ws = torch.zeros(nbytes, dtype=torch.uint8, device=self.device)
            self._batch_workspaces[cap] = ws
        table = (HqState * m)(*[st.struct for st in states])
        stream = self.stream
        stream.wait_stream(torch.cuda.current_stream(self.device))   # the workspace's zero fill
        for st in states:
            stream.wait_stream(st.stream)
        return table, cap, ws, stream

    def _batch_release(self, states, stream) -> None:
        for st in states:
            st.stream.wait_stream(stream)
        torch.cuda.current_stream(self.device).wait_stream(stream)

    def forward_tokens(self, token_ids, states) -> list[torch.Tensor]:
        """One decode step for each (token, state) pair of a batch of up to 32
        independent sequences: the reference's forward_token
        (cpu_lightspark.py:424-468) applied to each pair, with the same bits,
        in one hq_decode_batch call that reads every weight once for the
        whole batch.  Returns each state's logits (device tensors); each
        greedy token is left in its ``state.token``."""
        states = list(states)
        ids = [int(t) for t in token_ids]
        if len(ids) != len(states):
            raise ValueError("one token per decode state")
        for t, st in zip(ids, states):
            self._check_token(t, st)
        table, cap, ws, stream = self._batch_setup(states)
        with torch.cuda.stream(stream):
            for t, st in zip(ids, states):
                st.token.fill_(t)
        check(_native.lib().hq_decode_batch(ctypes.byref(self.struct), table, len(states), cap, ws.data_ptr(),
                                            stream.cuda_stream), "hq_decode_batch")
        for st in states:
            st.position += 1
        self._batch_release(states, stream)
        return [st.logits for st in states]

    def decode_greedy_batch(self, states, steps: int, use_graph: bool = True, check_status: bool = True) -> None:
        """`steps` batched greedy steps over the states, each feeding its
        argmax token back on the device (the tokens already in the states'
        ``token`` are consumed first), replayed from one captured HIP graph
        of the batched step.  With `check_status` the call waits and raises
        on any state's device status."""
        states = list(states)
        for st in states:
            if st.position + steps > st.capacity:
                raise ValueError("decode state capacity exhausted")
        table, cap, ws, stream = self._batch_setup(states)
        lib = _native.lib()
        if use_graph:
            # the graph holds the states' device pointers: it is kept with the
            # states themselves (so they outlive it) and only for this batch
            key = (tuple(bytes(st.struct) for st in states), cap)
            if self._batch_graph is None or self._batch_graph[0] != key:
                graph = torch.cuda.CUDAGraph()
                err = 0
                with torch.cuda.graph(graph, stream=stream):
                    err = lib.hq_decode_batch(ctypes.byref(self.struct), table, len(states), cap, ws.data_ptr(),
                                              stream.cuda_stream)
                check(err, "hq_decode_batch (graph capture)")
                self._batch_graph = (key, graph, states)
            graph = self._batch_graph[1]
            with torch.cuda.stream(stream):
                for _ in range(steps):
                    graph.replay()
        else:
            for _ in range(steps):
                check(lib.hq_decode_batch(ctypes.byref(self.struct), table, len(states), cap, ws.data_ptr(),
                                          stream.cuda_stream), "hq_decode_batch")
        for st in states:
            st.position += steps
        self._batch_release(states, stream)
        if check_status:
            for st in states:
                st.check_status()

    def decode_sampled(self, state: QwenDecodeState, steps: int, args, generator, generated) -> list[int]:
        """`steps` iterations of the reference's stochastic decode loop
        (cpu_lightspark.py:869-880) with no host round trip per token: each
        step forwards a token, samples the next one from its logits
        (hq_sample_token, the policy of `args`) and feeds it back on the
        device.

        `generated` is the run's list of generated tokens; its last entry is
        the token forwarded first (the reference appends a token before
        forwarding it), and the penalty of step i sees the list plus the i
        tokens sampled before.  Generator.choice consumes one
        generator.random() per token, so the `steps` draws are taken here up
        front, in the order the reference takes them.  Returns the sampled
        tokens (the last one is left in ``state.token``, not yet forwarded).
        The loop does not stop at end-of-turn tokens: the caller truncates.
        """
        if steps < 1:
            return []
        if state.position + steps > state.capacity:
            raise ValueError("decode state capacity exhausted")
        if len(generated) == 0:
            raise ValueError("generated must end with the token to forward")
        top_k = int(args.top_k)
        if not 1 <= top_k <= SAMPLE_MAX_TOP_K:
            raise ValueError(f"top_k must be in [1, {SAMPLE_MAX_TOP_K}] on the GPU sampler")
        if not (np.isfinite(args.temperature) and args.temperature > 0 and np.isfinite(args.top_p)
                and args.top_p > 0 and np.isfinite(args.repetition_penalty) and args.repetition_penalty > 0):
            raise ValueError("temperature, top_p and repetition_penalty must be positive and finite")
        vocab = int(self.config["vocab_size"])
        history = np.asarray(list(generated), dtype=np.int64).reshape(-1)
        if history.size and (history.min() < 0 or history.max() >= vocab):
            raise IndexError("a generated id is outside the vocabulary")
        n0 = int(history.size)
        lib = _native.lib()
        draws = np.array([generator.random() for _ in range(steps)], dtype=np.float64)
        dev = self.device
        with torch.cuda.stream(state.stream):
            gen = torch.empty(n0 + steps, dtype=torch.int32, device=dev)
            gen[:n0].copy_(torch.from_numpy(history.astype(np.int32)))
            state.token.copy_(gen[n0 - 1:n0])
            u = torch.from_numpy(draws).to(dev)
        ws = _zeroed_workspace(("sample", dev.index), lib.hq_sample_workspace_bytes(vocab, top_k), dev,
                               state.stream)
        model, st, stream = ctypes.byref(self.struct), ctypes.byref(state.struct), state.stream.cuda_stream
        for i in range(steps):
            check(lib.hq_decode_step(model, st, stream), "hq_decode_step")
            out = gen[n0 + i:n0 + i + 1]
            check(lib.hq_sample_token(state.logits.data_ptr(), vocab, gen.data_ptr(), n0 + i,
                                      float(args.repetition_penalty), float(args.temperature), top_k,
                                      float(args.top_p), u[i:].data_ptr(), out.data_ptr(), None, None,
                                      ws.data_ptr(), stream), "hq_sample_token")
            with torch.cuda.stream(state.stream):
                state.token.copy_(out)
        state.position += steps
        state.check_status()
        return [int(t) for t in gen[n0:].cpu().tolist()]

    # -- the reference's per-op surface ---------------------------------------
    def _projection(self, projection: LiteSparkProjection, values, quantized: torch.Tensor,
                    activation_scale: float, out: torch.Tensor,
                    stream: torch.cuda.Stream | None = None) -> None:
        """int8 activations x packed int4 weights (cpu_lightspark.py:351-371)."""
        if quantized.dtype != torch.int8 or quantized.numel() < projection.input_size:
            raise ValueError("quantized activations must be int8 [input_size]")
        if out.dtype != torch.float32 or out.numel() < projection.output_size:
            raise ValueError("output must be float32 [output_size]")
        check(_native.lib().hq_int4_i8_gemv(
            quantized.data_ptr(), projection.weights.data_ptr(), projection.scales.data_ptr(),
            float(activation_scale), out.data_ptr(), projection.output_size, projection.input_size,
            _stream_handle(stream)), "hq_int4_i8_gemv")

    def _attention(self, state: QwenDecodeState, layer_index: int) -> None:
        """GQA over the state's cache up to its position (cpu_lightspark.py:389-422),
        from ``state.q`` into ``state.attended``."""
        c = self.config
        kv_heads = int(c["num_key_value_heads"])
        groups = int(c["num_attention_heads"]) // kv_heads
        head_dim = int(c["head_dim"])
        end = state.position + 1
        gqa_decode(state.q, state.keys[layer_index], state.values[layer_index],
                   state.attended.view(-1, head_dim), end, kv_heads, groups, head_dim,
                   stream=state.stream)


def sample_logits(logits, generated, args, generator=None) -> int:
    """cpu_lightspark.py:700-726 on the device.

    argmax: the first maximal index (:704-705).  Otherwise the reference's
    policy (:706-726) through hq_sample_token; Generator.choice(ids, p)
    consumes one generator.random() draw, which is taken here on the host
    in the same place of the generator's stream and handed to the device.
    """
    if getattr(args, "argmax", False):
        return argmax(logits)
    if generator is None:
        raise ValueError("stochastic sampling needs the run's numpy Generator")
    token, _, _ = sample_token(logits, generated, args.repetition_penalty, args.temperature, args.top_k,
                               args.top_p, generator.random())
    return token


# --------------------------------------------------------------------------- ops
_workspaces: dict[tuple, torch.Tensor] = {}


def _zeroed_workspace(kind: tuple, nbytes: int, device, stream=None) -> torch.Tensor:
    """A zero-filled device workspace kept for reuse (the library returns the
    regions it needs zeroed to zero after every call).

    Workspaces are keyed by the stream the call runs on as well as by `kind`:
    calls on one stream run in order, while calls on two streams may overlap,
    and overlapping calls on one workspace would share its ticket counters.
    The zero fill runs on the current stream; a given `stream` is made to
    wait for it."""
    handle = (stream if stream is not None else torch.cuda.current_stream(device)).cuda_stream
    key = (*kind, handle)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    if stream is not None:
        stream.wait_stream(torch.cuda.current_stream(device))
    return ws


def quant_int4_gemv(x: torch.Tensor, projection: LiteSparkProjection, out: torch.Tensor | None = None,
                    q_out: torch.Tensor | None = None, act_out: torch.Tensor | None = None,
                    acc_out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Fused per-token int8 quantization + int4 GEMV (hq_quant_int4_gemv)."""
    if x.dtype != torch.float32 or x.numel() != projection.input_size or not x.is_contiguous():
        raise ValueError("x must be a contiguous float32 [input_size] device tensor")
    if out is None:
        out = torch.empty(projection.output_size, dtype=torch.float32, device=x.device)
    check(_native.lib().hq_quant_int4_gemv(
        x.data_ptr(), projection.weights.data_ptr(), projection.scales.data_ptr(), out.data_ptr(),
        projection.output_size, projection.input_size, _ptr(q_out), _ptr(act_out), _ptr(acc_out),
        _stream_handle(stream)), "hq_quant_int4_gemv")
    return out


def int4_i8_gemv(x_q: torch.Tensor, projection: LiteSparkProjection, activation_scale: float,
                 out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    if out is None:
        out = torch.empty(projection.output_size, dtype=torch.float32, device=x_q.device)
    check(_native.lib().hq_int4_i8_gemv(
        x_q.data_ptr(), projection.weights.data_ptr(), projection.scales.data_ptr(),
        float(activation_scale), out.data_ptr(), projection.output_size, projection.input_size,
        _stream_handle(stream)), "hq_int4_i8_gemv")
    return out


def quantize_activation(x: torch.Tensor, q: torch.Tensor | None = None, stream=None):
    """Per-token int8 quantization on the device; returns (q, act_scale tensor[1])."""
    if q is None:
        q = torch.empty(x.numel(), dtype=torch.int8, device=x.device)
    act = torch.empty(1, dtype=torch.float32, device=x.device)
    check(_native.lib().hq_quantize_activation(x.data_ptr(), x.numel(), q.data_ptr(), act.data_ptr(),
                                               _stream_handle(stream)), "hq_quantize_activation")
    return q, act


def rmsnorm(x: torch.Tensor, gamma: torch.Tensor, eps: float, out: torch.Tensor | None = None,
            stream=None) -> torch.Tensor:
    if out is None:
        out = torch.empty_like(x)
    check(_native.lib().hq_rmsnorm(x.data_ptr(), gamma.data_ptr(), out.data_ptr(), x.numel(), float(eps),
                                   _stream_handle(stream)), "hq_rmsnorm")
    return out


def gqa_decode(query: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, out: torch.Tensor,
               context: int, kv_heads: int, groups: int, head_dim: int, stream=None) -> torch.Tensor:
    """Fused GQA decode over an fp16 [capacity, kv_heads, head_dim] cache
    (hq_gqa_decode, the reference's litespark_gqa_decode call at
    cpu_lightspark.py:394-406 with score_stride = the cache's capacity)."""
    if keys.dtype != torch.float16 or values.dtype != torch.float16:
        raise ValueError("keys/values must be float16")
    shape = (keys.shape[0], kv_heads, head_dim)
    if (keys.dim() != 3 or tuple(keys.shape) != shape or tuple(values.shape) != shape
            or not keys.is_contiguous() or not values.is_contiguous()):
        raise ValueError("keys/values must be contiguous float16 [capacity, kv_heads, head_dim]")
    capacity = int(keys.shape[0])
    if context < 1 or context > capacity:
        raise ValueError("context outside the cache")
    lib = _native.lib()
    nbytes = lib.hq_gqa_workspace_bytes(capacity, kv_heads, groups, head_dim)
    ws = _zeroed_workspace(("gqa", query.device.index), nbytes, query.device, stream)
    check(lib.hq_gqa_decode(query.data_ptr(), keys.data_ptr(), values.data_ptr(), ws.data_ptr(),
                            out.data_ptr(), context, kv_heads, groups, head_dim,
                            capacity, _stream_handle(stream)), "hq_gqa_decode")
    return out


def int4_i8_gemm(x_q: torch.Tensor, act_scales: torch.Tensor, projection: LiteSparkProjection,
                 out: torch.Tensor | None = None, acc_out: torch.Tensor | None = None,
                 stream=None) -> torch.Tensor:
    """M sequences x one int4 matrix on int8 MFMA (hq_int4_i8_gemm)."""
    m = x_q.shape[0]
    if out is None:
        out = torch.empty((m, projection.output_size), dtype=torch.float32, device=x_q.device)
    lib = _native.lib()
    nbytes = lib.hq_gemm_workspace_bytes(m, projection.output_size, projection.input_size)
    ws = _zeroed_workspace(("gemm", x_q.device.index, m, projection.output_size,
                            projection.input_size), nbytes, x_q.device, stream)
    check(lib.hq_int4_i8_gemm(x_q.data_ptr(), act_scales.data_ptr(), projection.weights.data_ptr(),
                              projection.scales.data_ptr(), out.data_ptr(), m, projection.output_size,
                              projection.input_size, _ptr(acc_out), ws.data_ptr(),
                              _stream_handle(stream)), "hq_int4_i8_gemm")
    return out


def quant_int4_gemm(x: torch.Tensor, projection: LiteSparkProjection, out: torch.Tensor | None = None,
                    q_out=None, act_out=None, acc_out=None, stream=None) -> torch.Tensor:
    """Per-sequence quantization + int4 GEMM on int8 MFMA (hq_quant_int4_gemm)."""
    m = x.shape[0]
    if out is None:
        out = torch.empty((m, projection.output_size), dtype=torch.float32, device=x.device)
    lib = _native.lib()
    nbytes = lib.hq_gemm_workspace_bytes(m, projection.output_size, projection.input_size)
    ws = _zeroed_workspace(("gemm", x.device.index, m, projection.output_size,
                            projection.input_size), nbytes, x.device, stream)
    check(lib.hq_quant_int4_gemm(x.data_ptr(), projection.weights.data_ptr(), projection.scales.data_ptr(),
                                 out.data_ptr(), m, projection.output_size, projection.input_size,
                                 _ptr(q_out), _ptr(act_out), _ptr(acc_out), ws.data_ptr(),
                                 _stream_handle(stream)), "hq_quant_int4_gemm")
    return out


def argmax(logits: torch.Tensor, stream=None) -> int:
    """First maximal index, as np.argmax (cpu_lightspark.py:704-705), on the device."""
    if logits.dtype != torch.float32 or not logits.is_cuda or not logits.is_contiguous():
        raise ValueError("logits must be a contiguous float32 device tensor")
    lib = _native.lib()
    n = logits.numel()
    ws = _zeroed_workspace(("argmax", logits.device.index), lib.hq_argmax_workspace_bytes(n),
                           logits.device, stream)
    out = torch.empty(1, dtype=torch.int32, device=logits.device)
    check(lib.hq_argmax(logits.data_ptr(), n, out.data_ptr(), ws.data_ptr(), _stream_handle(stream)),
          "hq_argmax")
    if stream is not None:
        stream.synchronize()
    return int(out.item())


SAMPLE_MAX_TOP_K = 2048


def sample_token(logits: torch.Tensor, generated, repetition_penalty: float, temperature: float, top_k: int,
                 top_p: float, u: float, stream=None):
    """One draw of the reference's stochastic policy (cpu_lightspark.py:706-726)
    given the uniform number u in [0, 1): returns (token, ids, probabilities)
    with the ranked top-k ids and their final probabilities as host arrays.

    generated ids index the logits as numpy does (a negative id counts from
    the end; one outside [-n, n) raises IndexError).
    """
    if logits.dtype != torch.float32 or not logits.is_cuda or not logits.is_contiguous():
        raise ValueError("logits must be a contiguous float32 device tensor")
    n = logits.numel()
    if not 1 <= int(top_k) <= SAMPLE_MAX_TOP_K:
        raise ValueError(f"top_k must be in [1, {SAMPLE_MAX_TOP_K}] on the GPU sampler")
    if not (np.isfinite(temperature) and temperature > 0):
        raise ValueError("temperature must be positive and finite")
    if not (np.isfinite(top_p) and top_p > 0):
        raise ValueError("top_p must be positive")
    if not (np.isfinite(repetition_penalty) and repetition_penalty > 0):
        raise ValueError("repetition_penalty must be positive")
    if not 0.0 <= float(u) < 1.0:
        raise ValueError("u must be in [0, 1)")
    ids = np.asarray(list(generated) if generated is not None else [], dtype=np.int64).reshape(-1)
    if ids.size and (ids.min() < -n or ids.max() >= n):
        raise IndexError("a generated id is outside the logits")
    ids = np.where(ids < 0, ids + n, ids).astype(np.int32)
    device = logits.device
    k = min(int(top_k), n)
    lib = _native.lib()
    ws = _zeroed_workspace(("sample", device.index), lib.hq_sample_workspace_bytes(n, k), device, stream)
    gen = torch.from_numpy(ids).to(device) if ids.size else None
    draw = torch.tensor([float(u)], dtype=torch.float64, device=device)
    out = torch.empty(1, dtype=torch.int32, device=device)
    ranked = torch.empty(k, dtype=torch.int32, device=device)
    probs = torch.empty(k, dtype=torch.float32, device=device)
    check(lib.hq_sample_token(logits.data_ptr(), n, _ptr(gen), int(ids.size), float(repetition_penalty),
                              float(temperature), int(top_k), float(top_p), draw.data_ptr(), out.data_ptr(),
                              ranked.data_ptr(), probs.data_ptr(), ws.data_ptr(), _stream_handle(stream)),
          "hq_sample_token")
    if stream is not None:
        stream.synchronize()
    return int(out.item()), ranked.cpu().numpy(), probs.cpu().numpy()
