"""Per-category profile of one decode token on the GPU.

This is the counterpart of the reference's profile_forward_token
(cpu_lightspark.py:470-553, printed at :851-857 of the reference repository;
its table is in README.md:102-116 there).  The reference times every kernel
call of one forward_token on the CPU and sums the times into categories:
body GEMV, attention, activation quantization, norms, embedding + LM head.

On the GPU the 36 decoder layers of a step run as one persistent kernel, so
the categories are read from inside it.  The HQ_ENGINE_TRACE build
(libhq_trace.so, from `python -m harsh4b_amd.build --trace`) records a
timestamp at every phase boundary of layers 16-19 in every block.  A layer's
critical path is a chain of these points, and each segment between two
points goes to one category:
  - GEMV dots (weights in registers): the weight waves' dot products over
    weights already loaded (their streaming overlaps the other segments, so
    this is not the reference's body-GEMV time, which includes the loads);
  - attention: an attention item, from its inputs to its output;
  - norm + quant: the RMSNorm and quantization prologues;
  - hand-off: the cross-block hand-offs (watching a vector's last entry,
    then reading the vector);
  - sync: passing work between the block's input and weight waves.
The segment lengths are block medians, and they add up to the layer's
median time.  They are scaled by the untraced/traced layer-kernel time
ratio (the trace costs a few percent) and multiplied by the number of
layers.  The rest of the step is embedding + LM head + argmax: the step's
time minus the layer kernel's.  Sampling is one hq_sample_token launch with
the reference runtime's policy (penalty 1.15, temperature 0.7, top-k 50,
top-p 0.9) over the step's logits, as decode_sampled runs it on the device.

Run (libhq.so and libhq_trace.so built):
    python -m harsh4b_amd.profile [--ctx 64] [--json]

The orchestrating process runs the two measurements as child processes
(`--part trace` on libhq_trace.so, `--part time` on libhq.so) and does not
touch the GPU itself.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import subprocess
import sys
from pathlib import Path

from . import _native, build

TRACE_L0, TRACE_LAYERS, TRACE_POINTS = 16, 4, 96     # kTraceL0, layers, kTracePoints (hq_engine.hip)
TRACE_BLOCKS = 1024                                  # blocks the trace buffer holds

# A layer's critical path: (from point, to point, category, what).  Points
# 25-29 are taken in the blocks that ran an attention item; "end" is the
# next layer's point 0.
DOTS = "GEMV dots (weights in registers)"
SEGMENTS = [
    (0, 2, "hand-off", "x (layer input): watch + read"),
    (2, 3, "norm + quant", "RMSNorm + quant, qkv input"),
    (3, 16, "sync", "qkv input -> weight waves"),
    (16, 4, DOTS, "qkv (dot, rows to the input waves)"),
    (4, 25, "hand-off", "qkv rows -> attention items"),
    (25, 29, "attention", "attention item (norms, RoPE, scores, softmax, V)"),
    (29, 6, "hand-off", "attention output: watch"),
    (6, 7, "hand-off", "attention output: read + quant"),
    (7, 18, "sync", "o input -> weight waves"),
    (18, 8, DOTS, "o (dot, rows to the input waves)"),
    (8, 9, "hand-off", "x + o (residual): watch"),
    (9, 32, "hand-off", "x + o (residual): read"),
    (32, 10, "norm + quant", "RMSNorm + quant, gate_up input"),
    (10, 20, "sync", "gate_up input -> weight waves"),
    (20, 11, DOTS, "gate_up + SwiGLU (dot, rows to the input waves)"),
    (11, 12, "hand-off", "SwiGLU output: watch"),
    (12, 42, "hand-off", "SwiGLU output: read + max"),
    (42, 44, "norm + quant", "quant, down input"),
    (44, 22, "sync", "down input -> weight waves"),
    (22, 14, DOTS, "down (dot, rows to the input waves)"),
    (14, "end", "hand-off", "residual store -> next layer"),
]
ATTENTION_POINTS = {25, 26, 27, 28, 29, 48, 49, 50, 51, 52, 53}
# Past 256 positions the attention runs as GQA items (kv head, group of
# chunks: points 48-53, taken in the blocks that ran one) and a combine
# spread over every block (points 54-56).
GQA_SEGMENTS = [s for s in SEGMENTS if s[0] not in (4, 25, 29)]
GQA_SEGMENTS[GQA_SEGMENTS.index((6, 7, "hand-off", "attention output: read + quant")):
             GQA_SEGMENTS.index((6, 7, "hand-off", "attention output: read + quant"))] = [
    (4, 49, "hand-off", "qkv rows -> GQA items (q/k rows in)"),
    (49, 50, "attention", "GQA item: q/k prologue, K/V copies landed"),
    (50, 51, "attention", "GQA item: scores (4 query heads)"),
    (51, 53, "attention", "GQA item: softmax, V, partials published"),
    (53, 55, "hand-off", "chunk partials -> every block (gather)"),
    (55, 56, "attention", "combine (M, a_c, L/O chains)"),
    (56, 6, "hand-off", "attention output: watch"),
]
CATEGORIES = [DOTS, "attention", "norm + quant", "hand-off", "sync"]


def _model_and_state(ctx, seed, extra):
    import numpy as np
    from .config import QWEN3_4B
    from .synthetic import random_model
    model = random_model(QWEN3_4B, seed=seed)
    state = model.new_state(ctx + 16 + extra + 8)
    prompt = [int(t) for t in np.random.default_rng(3).integers(0, int(QWEN3_4B["vocab_size"]), ctx)]
    model.prefill(prompt, state)
    model.decode_greedy(state, 16)
    state.synchronize()
    return model, state


def part_trace(ctx, seed, reps=4):
    """Segment medians (us, traced clock) of layers 16-18 at context ctx+17."""
    import numpy as np
    import torch
    _native.LIB_PATH = build.TRACE_LIB
    lib = _native.lib()
    model, state = _model_and_state(ctx, seed, 0)
    s = state.stream
    words = TRACE_LAYERS * TRACE_POINTS
    nb = model.layer_kernel_blocks() if callable(model.layer_kernel_blocks) else model.layer_kernel_blocks
    traces = []
    for _ in range(reps):
        _native.check(lib.hq_step_layers(ctypes.byref(model.struct), ctypes.byref(state.struct), s.cuda_stream),
                      "hq_step_layers")
        torch.cuda.synchronize()
        raw = state.workspace[-TRACE_BLOCKS * words * 4:].view(torch.int32).cpu().numpy()
        traces.append(raw.view(np.uint32).reshape(TRACE_BLOCKS, TRACE_LAYERS, TRACE_POINTS)[:nb].astype(np.int64))
    state.check_status()
    tr = traces[-1]
    has_att = (tr[:, 0, 25] != 0) & (tr[:, 0, 29] != 0)
    segments = SEGMENTS if has_att.any() else GQA_SEGMENTS
    if not has_att.any():
        has_att = (tr[:, 0, 48] != 0) & (tr[:, 0, 53] != 0)     # the blocks that ran a GQA item
    per_layer = []
    for L in range(TRACE_LAYERS - 1):
        # every block's points from one origin, the median layer start (the
        # blocks that run attention items start a layer earlier than the
        # others: they hold no hidden rows); a point's median is taken over
        # the blocks that recorded it (a block that skips a phase leaves 0)
        origin = np.median(tr[:, L, 0])
        rel = (tr[:, L, :] - origin) / 100.0                   # 100 MHz clock -> us
        end = (tr[:, L + 1, 0] - tr[:, L, 0]) / 100.0

        def med(point):
            if point == "end":
                return float((np.median(tr[:, L + 1, 0]) - origin) / 100.0)
            sel = tr[:, L, point] != 0
            if point in ATTENTION_POINTS:
                sel &= has_att
            return float(np.median(rel[sel, point]))
        segs = [(a, b, cat, what, med(b) - med(a)) for a, b, cat, what in segments]
        per_layer.append({"layer": TRACE_L0 + L, "us": float(np.median(end)), "segments": segs})
    return {"context": int(state.device_position.item()) + 1, "blocks": nb,
            "attention_blocks": int(has_att.sum()), "layers": per_layer}


def part_time(ctx, seed, steps=64):
    """Untraced times: layer kernel per launch, decode step, sampler."""
    import numpy as np
    import torch
    lib = _native.lib()
    model, state = _model_and_state(ctx, seed, steps)
    s = state.stream
    context = int(state.device_position.item()) + 1

    def timed(fn, n):
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(n):
            fn()
        e1.record(s)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / n

    cap = torch.cuda.CUDAGraph()
    with torch.cuda.graph(cap, stream=s):
        for _ in range(4):
            _native.check(lib.hq_step_layers(ctypes.byref(model.struct), ctypes.byref(state.struct),
                                             s.cuda_stream), "hq_step_layers")
    with torch.cuda.stream(s):
        cap.replay()
        layers_us = min(timed(cap.replay, 5) for _ in range(3)) / 4
    del cap
    step_us = timed(lambda: model.decode_greedy(state, steps, check_status=False), 1) / steps
    state.check_status()
    logits = state.logits
    n = logits.numel()
    dev = logits.device
    ids = torch.from_numpy(np.random.default_rng(1).integers(0, n, 64).astype(np.int32)).to(dev)
    u = torch.tensor([0.5], dtype=torch.float64, device=dev)
    out = torch.empty(1, dtype=torch.int32, device=dev)
    ws = torch.zeros(lib.hq_sample_workspace_bytes(n, 50), dtype=torch.uint8, device=dev)

    def sample():
        _native.check(lib.hq_sample_token(logits.data_ptr(), n, ids.data_ptr(), 64, 1.15, 0.7, 50, 0.9,
                                          u.data_ptr(), out.data_ptr(), None, None, ws.data_ptr(),
                                          s.cuda_stream), "hq_sample_token")
    sample()
    sample_us = timed(sample, 32)
    return {"context": context, "layers_us": layers_us, "step_us": step_us, "sample_us": sample_us}


def combine(tr, tm, layers=36):
    traced_layer = sum(l["us"] for l in tr["layers"]) / len(tr["layers"])
    scale = (tm["layers_us"] / layers) / traced_layer
    cats = {c: 0.0 for c in CATEGORIES}
    rows = {}
    for l in tr["layers"]:
        for a, b, cat, what, us in l["segments"]:
            cats[cat] += us / len(tr["layers"])
            rows[what] = rows.get(what, 0.0) + us / len(tr["layers"])
    token = {c: v * scale * layers for c, v in cats.items()}
    token["embedding + LM head + argmax"] = tm["step_us"] - tm["layers_us"]
    token["sampling (hq_sample_token)"] = tm["sample_us"]
    total = tm["step_us"] + tm["sample_us"]
    return {"context": tm["context"], "layer_kernel_us": round(tm["layers_us"], 1),
            "step_us": round(tm["step_us"], 1), "traced_layer_us": round(traced_layer, 2),
            "trace_scale": round(scale, 4), "attention_blocks": tr["attention_blocks"],
            "token_us": {k: round(v, 1) for k, v in token.items()},
            "token_share": {k: round(v / total, 4) for k, v in token.items()},
            "layer_segments_us": {k: round(v * scale, 3) for k, v in rows.items()}}


def markdown(res):
    out = [f"Decode token at context {res['context']}: step {res['step_us']:.1f} us "
           f"(layer kernel {res['layer_kernel_us']:.1f} us) + sampling.", "",
           "| category | us per token | share |", "|---|---:|---:|"]
    for k, v in res["token_us"].items():
        out.append(f"| {k} | {v:.1f} | {100 * res['token_share'][k]:.1f} % |")
    out += ["", "Per layer (critical path, block medians, scaled to the untraced kernel):", "",
            "| segment | us |", "|---|---:|"]
    for k, v in res["layer_segments_us"].items():
        out.append(f"| {k} | {v:.3f} |")
    return "\n".join(out)


def main(argv=None):
    ap = argparse.ArgumentParser(description="per-category profile of one decode token")
    ap.add_argument("--ctx", type=int, default=64, help="prompt tokens before the 16 warm-up steps")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--part", choices=("trace", "time"))
    ap.add_argument("--json", action="store_true")
    args = ap.parse_args(argv)
    if args.part == "trace":
        print(json.dumps(part_trace(args.ctx, args.seed)))
        return
    if args.part == "time":
        print(json.dumps(part_time(args.ctx, args.seed)))
        return
    for lib in (build.LIB, build.TRACE_LIB):
        if not lib.exists():
            raise SystemExit(f"{lib} is missing: python -m harsh4b_amd.build --trace")
    parts = {}
    for part in ("trace", "time"):
        r = subprocess.run([sys.executable, "-m", "harsh4b_amd.profile", "--part", part, "--ctx", str(args.ctx),
                            "--seed", str(args.seed)], capture_output=True, text=True,
                           cwd=str(Path(__file__).resolve().parent.parent))
        if r.returncode != 0:
            sys.stderr.write(r.stderr)
            raise SystemExit(f"profile part {part} failed ({r.returncode})")
        parts[part] = json.loads(r.stdout.strip().splitlines()[-1])
    res = combine(parts["trace"], parts["time"])
    print(json.dumps(res, indent=1) if args.json else markdown(res))


if __name__ == "__main__":
    main()
