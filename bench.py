#!/usr/bin/env python3
"""Decode benchmark of the int4 hot path on one MI355X.

Workload: a random-init 36-layer Qwen3-4B-shaped
int4 model (hidden 2560, 32 q / 8 kv heads x 128, SwiGLU 9728, tied int4
embedding/LM head 151936 x 2560), fp16 KV cache, batch 1, greedy decoding
after a 64-token random prompt.  A "step" is one decode token: 144 body
GEMVs + 36 attentions + LM head + argmax, replayed from a HIP graph with the
greedy token fed back on the device.

Printed as one JSON line: tok/s (value); the HBM roofline of the dominant
kernel, the persistent layer kernel that runs all 36 decoder layers of a step
in one launch (about 95 % of the step time), timed live with HIP events on
its launch stream; the body-weight bandwidth of that launch; and, under
"configs", the other BASELINE configurations measured in the same run, each
with its own roofline and CPU baseline: configs[0] (one fused quant + int4
GEMV 2560 -> 9728 over rotating weight copies), configs[1] (one decoder
layer's body GEMVs: the standalone GEMV kernels and the layer kernel's
per-layer share), configs[4] (the same decode at context 4096, with the
attention's KV bandwidth) and configs[3] (the batched decode step of M = 8
and 32 sequences at context 256).  cpu_baseline is the CPU oracle (this repository's
C restatement of the reference path; AVX-512 VNNI GEMVs where the host has
them) decoding the same model on this host, on all available cores and on
the reference's default 6 threads, with the CPU model and core counts.
`roofline.traffic` is the layer kernel's HBM bytes per launch at the line's
own context from the committed PMC profile (profiles/engine_traffic_pmc.json,
made with --workload layers under rocprofv3 --pmc and --pmc-summary), or null
when no profile holds that context.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
TRAFFIC_PROFILE = ROOT / "profiles" / "engine_traffic_pmc.json"
REFERENCE_THREADS = 6          # the reference runner's default (cpu_lightspark.py:34, 38-42)
METRIC = "decode tok/s @ Qwen3-4B batch 1; body-GEMV HBM GB/s as % of peak"
# The reference's published decode rates for this model at batch 1, 256
# tokens (README.md:139-144 of the reference repository, Apple M4 CPU, 6
# threads): greedy 33.17-35.02 tok/s (the top of the range is used), default
# stochastic sampler 33.65 tok/s.
PUBLISHED_GREEDY_TOK_S = 35.02
PUBLISHED_SAMPLED_TOK_S = 33.65


def parse():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--ctx", type=int, default=None,
                    help="context before the timed decode (default 64; 4096 for --workload long)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--gemv-reps", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="CPU time of each decode baseline run (the GEMV runs take a quarter of it)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--batch-fill", action="store_true",
                    help="batched workload: fill each sequence's cache with N(0,1) K/V instead of prefilling "
                         "its prompt (the PMC runs then see only the decode step's kernels)")
    ap.add_argument("--pmc-kernels", nargs=5, metavar=("MFMA_DIR", "FETCH_DIR", "WRITE_DIR", "COPY_FETCH_DIR",
                                                       "COPY_WRITE_DIR"),
                    help="fold rocprofv3 --pmc runs of one workload into per-kernel MFMA utilisation, int8 "
                         "TOP/s and HBM bytes (MFMA_DIR: SQ_INSTS_VALU_MFMA_MOPS_I8, SQ_VALU_MFMA_BUSY_CYCLES, "
                         "GRBM_GUI_ACTIVE; FETCH_DIR: FETCH_SIZE; WRITE_DIR: WRITE_SIZE; COPY_*: the same "
                         "counters over --workload copy)")
    ap.add_argument("--batch-sizes", default="8,16,32",
                    help="batched: comma-separated M values; value is the largest M's rate")
    ap.add_argument("--no-configs", action="store_true",
                    help="decode: skip the configs[0]/[1]/[3]/[4] measurements folded into the line")
    ap.add_argument("--pmc-summary", nargs=4, metavar=("FETCH_DIR", "WRITE_DIR", "COPY_FETCH_DIR", "COPY_WRITE_DIR"),
                    help="print the traffic summary of rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE output "
                         "directories of --workload layers and --workload copy runs")
    ap.add_argument("--workload", choices=("decode", "sampled", "sample", "long", "batched", "gemv", "copy",
                                           "layers", "attention"),
                    default="decode",
                    help="decode: configs[2] (the reported line); sampled: the same decode with the "
                         "reference runner's default stochastic sampler (temperature 0.7, top-k 40, "
                         "top-p 0.9, repetition penalty 1.08) on the GPU; sample: that sampler alone, per "
                         "top-k; long: configs[4], the same decode "
                         "at context 4096 over an N(0,1) fp16 KV cache; batched: configs[3], the "
                         "body GEMMs of M = 8/16/32 sequences on int8 MFMA against M GEMVs; attention: the "
                         "standalone hq_gqa_decode at --ctx (default 4096); gemv: "
                         "configs[0], one fused quant + int4 GEMV 2560 -> 9728 over rotating weight "
                         "copies; copy: a plain 256 MiB device-to-device copy, the calibration kernel "
                         "of the PMC traffic counters; layers: the layer kernel alone, launched "
                         "--steps times at the default line's context (or --ctx with the long workload's "
                         "N(0,1) cache), for rocprofv3 --pmc")
    return ap.parse_args()


def algorithmic_bytes(config):
    """Bytes one launch of each body GEMV kind must move (weights + scales +
    fp32 activations in + fp32 outputs + norm weights)."""
    from harsh4b_amd.config import shapes
    sh = shapes(config)
    h = int(config["hidden_size"])
    i = int(config["intermediate_size"])
    q = int(config["num_attention_heads"]) * int(config["head_dim"])
    out = {}
    r, w = sh["qkv"]
    out["qkv"] = r * w // 2 + 4 * r + 4 * w + 4 * w + 4 * r          # W, scales, x, gamma, out
    r, w = sh["o"]
    out["o"] = r * w // 2 + 4 * r + 4 * q + 4 * r + 4 * r             # W, scales, attended, x r+w
    r, w = sh["gate_up"]
    out["gate_up"] = r * w // 2 + 4 * r + 4 * w + 4 * w + 4 * i       # W, scales, x, gamma, act
    r, w = sh["down"]
    out["down"] = r * w // 2 + 4 * r + 4 * i + 4 * h + 4 * h          # W, scales, act, x r+w
    return out


def layer_kernel_bytes(config, context):
    """Algorithmic bytes of one launch of the persistent layer kernel (all
    decoder layers of a step) at `context` positions: packed body weights,
    row scales, norm weights, the K/V rows of the context-1 earlier positions
    (fp16) read by attention, the new K/V row written, the RoPE table rows
    and the residual vector in and out."""
    from harsh4b_amd.config import body_bytes, shapes
    L = int(config["num_hidden_layers"])
    h = int(config["hidden_size"])
    d = int(config["head_dim"])
    kvh = int(config["num_key_value_heads"])
    scales = 4 * L * sum(r for r, _ in shapes(config).values())
    norms = 4 * L * (2 * h + 2 * d)
    kv_row = 2 * kvh * d * 2                       # K and V of one position, fp16
    kv = L * kv_row * (context - 1) + L * kv_row
    rope = 4 * L * d
    return body_bytes(config) + scales + norms + kv + rope + 2 * 4 * h


def traffic_at(context):
    """HBM bytes per launch of the layer kernel at `context` from the PMC
    profile (FETCH_SIZE + WRITE_SIZE scaled by a copy kernel's reading), or
    None when the profile holds no run at exactly that context."""
    try:
        prof = json.loads(TRAFFIC_PROFILE.read_text())
    except (OSError, ValueError):
        return None
    for run in prof.get("runs", []):
        if int(run.get("context", -1)) == int(context):
            return int(run["traffic_bytes"])
    return None


def time_graph(lib, model, state, launches, reps, torch):
    """Capture `launches` (list of (layer, kind)) into a HIP graph on the
    state's stream, replay it `reps` times between two HIP events and
    return the mean time of one replay in ms."""
    s = state.stream
    err = 0
    torch.cuda.synchronize()
    cap = torch.cuda.CUDAGraph()
    with torch.cuda.graph(cap, stream=s):
        for layer, kind in launches:
            err |= lib.hq_step_gemv(ctypes.byref(model.struct), ctypes.byref(state.struct),
                                    layer, kind, s.cuda_stream)
    if err:
        raise RuntimeError("hq_step_gemv failed during capture")
    with torch.cuda.stream(s):       # replay() launches on the current stream
        cap.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            cap.replay()
        e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def time_layers(lib, model, state, launches, reps, torch):
    """Mean time (ms) of one launch of the step's decoder layers (the
    persistent layer kernel), from a HIP graph of `launches` launches
    replayed `reps` times between two HIP events on the launch stream."""
    s = state.stream
    torch.cuda.synchronize()
    cap = torch.cuda.CUDAGraph()
    err = 0
    with torch.cuda.graph(cap, stream=s):
        for _ in range(launches):
            err |= lib.hq_step_layers(ctypes.byref(model.struct), ctypes.byref(state.struct), s.cuda_stream)
    if err:
        raise RuntimeError("hq_step_layers failed during capture")
    with torch.cuda.stream(s):
        cap.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            cap.replay()
        e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (reps * launches)


def body_gemv_metric(cfg, per_kind_ms, layers_ms):
    """The body-GEMV bandwidth as the metric is defined: the packed body
    weight bytes of one token (1,816,657,920 at Qwen3-4B) over the summed
    durations of the token's body-GEMV kernels.  Those are separate kernels
    only in the five-kernels-per-layer form (36 x qkv, o, gate_up, down, each
    with its fused norm/quant prologue and epilogue, timed from graphs of
    each kind's 36 launches); in the fused step they share one persistent
    launch with attention, norms and hand-offs, and the weight stream cannot
    be timed apart, so that launch's figure (body bytes over its whole time,
    a lower bound) is given beside it."""
    from harsh4b_amd.config import body_bytes
    L = int(cfg["num_hidden_layers"])
    nbytes = body_bytes(cfg)
    us = L * sum(per_kind_ms.values()) * 1e3
    gbs = nbytes / (us * 1e-6) / 1e9
    fused_gbs = nbytes / (layers_ms * 1e-3) / 1e9
    return {"bytes_per_token": nbytes, "us_per_token": round(us, 2), "achieved": round(gbs, 1), "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "kernels": "gemv_rr_kernel (qkv, o, down) + gemv_kernel (gate_up), 144 per token (five-kernels-per-layer form)",
            "fused_step": {"us_per_token": round(layers_ms * 1e3, 2), "achieved": round(fused_gbs, 1),
                           "frac": round(fused_gbs / HBM_PEAK_GBS, 4),
                           "note": "body weight bytes / the persistent layer kernel's whole time (attention, "
                                   "norms and hand-offs included)"}}


def sampled_case(model, prompt, steps, warmup, seed):
    """The same decode with the reference runner's default stochastic
    sampler (temperature 0.7, top-k 40, top-p 0.9, repetition penalty 1.08;
    cpu_lightspark.py:706-726) on the GPU: a fresh state prefilled with the
    prompt, `warmup` sampled steps, then `steps` timed with HIP events."""
    import numpy as np
    import torch
    from types import SimpleNamespace
    from harsh4b_amd.lightspark import sample_logits
    policy = SimpleNamespace(argmax=False, temperature=0.7, top_k=40, top_p=0.9, repetition_penalty=1.08)
    generator = np.random.default_rng(seed)
    state = model.new_state(len(prompt) + warmup + steps + 4)
    model.prefill(prompt, state)
    generated = [sample_logits(state.logits, [], policy, generator)]
    generated += model.decode_sampled(state, warmup, policy, generator, generated)
    state.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(state.stream)
    generated += model.decode_sampled(state, steps, policy, generator, generated)
    e1.record(state.stream)
    torch.cuda.synchronize()
    state.check_status()
    tok_s = steps / (e0.elapsed_time(e1) / 1e3)
    return {"workload": "configs[2] with the reference runner's default stochastic sampler on the GPU "
                        f"(temperature 0.7, top-k 40, top-p 0.9, repetition penalty 1.08, seed {seed})",
            "tok_s": round(tok_s, 2), "steps": steps, "warmup": warmup,
            "vs_baseline": round(tok_s / PUBLISHED_SAMPLED_TOK_S, 2),
            "baseline": f"{PUBLISHED_SAMPLED_TOK_S} tok/s (the reference's published default-sampler decode rate)"}


def cpu_info():
    """CPU model, logical CPUs this process may run on, and the host's
    physical cores (distinct physical id / core id pairs)."""
    model, cores, phys = None, set(), None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key, val = key.strip(), val.strip()
                if key == "model name" and model is None:
                    model = val
                elif key == "physical id":
                    phys = val
                elif key == "core id":
                    cores.add((phys, val))
    except OSError:
        pass
    return {"cpu_model": model, "logical_cpus_available": len(os.sched_getaffinity(0)),
            "physical_cores_host": len(cores) or None}


def all_threads():
    """The cores this process has: its CPU affinity, capped by OMP_NUM_THREADS
    where that is set (the GPU box sets it to the job's CPU share)."""
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    return min(n, int(env)) if env.isdigit() and int(env) > 0 else n


def cpu_runs(run, seconds, unit, sample, kind="port"):
    """`run(seconds)` -> (value, detail) on all available cores and on the
    reference's 6 threads; the all-core run is the reported baseline."""
    import oracle
    out = {}
    for name, threads in (("all_cores", all_threads()), ("reference_threads", REFERENCE_THREADS)):
        oracle.set_threads(threads)
        value, detail = run(seconds)
        out[name] = {"threads": threads, "value": round(value, 3), "sample": detail}
    oracle.set_threads(all_threads())
    top = out["all_cores"]
    return {"value": top["value"], "unit": unit, "cores": top["threads"], "kind": kind,
            "sample": sample + "; " + top["sample"], "runs": out, "simd": "avx512-vnni" if oracle.simd_active()
            else "scalar", **cpu_info()}


CPU_WARMUP_TOKENS = 8   # the reference's decode rate skips 8 warm-up tokens (cpu_lightspark.py:735, 882-890)


def oracle_decode_rate(ref, state, ctx, seconds, token=1000):
    """tok/s of the oracle decoding from a cache of `ctx` positions after
    CPU_WARMUP_TOKENS untimed tokens (the position is reset before the run,
    so every run sees the same context); the state's capacity must leave
    room for the warm-up and the timed tokens."""
    state.position = ctx
    for _ in range(CPU_WARMUP_TOKENS):
        token = ref.forward_token(token, state)
    n, t0 = 0, time.perf_counter()
    while True:
        token = ref.forward_token(token, state)
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds and n >= 2) or state.position >= state.struct.capacity:
            break
    return n / el, f"{n} steps in {el:.1f} s"


def cpu_baseline(ref, state, ctx, seconds):
    """The CPU oracle (C restatement of the reference path) decoding from the
    same model and KV cache on this host."""
    def run(sec):
        return oracle_decode_rate(ref, state, ctx, sec)
    return cpu_runs(run, seconds, "tok/s", f"decode steps of the same 36-layer model at context {ctx}+, "
                                          "OpenMP over GEMV rows (oracle/hq_oracle.c)")


def oracle_state_from(ref, state, ctx, capacity):
    """An oracle state holding the first ctx cache positions of a device state."""
    import numpy as np
    rs = ref.new_state(capacity)
    rs.keys[:, :ctx] = state.keys[:, :ctx].cpu().numpy().view(np.uint16)
    rs.values[:, :ctx] = state.values[:, :ctx].cpu().numpy().view(np.uint16)
    rs.position = ctx
    return rs


GEMV_ROWS, GEMV_WIDTH, GEMV_COPIES = 9728, 2560, 48


def gemv_case(args, cpu_seconds):
    """fused per-token quant + int4 GEMV, K=2560 -> N=9728, with
    48 distinct weight copies (598 MB, above the 256 MB Infinity Cache)
    cycled so every launch streams its weights from HBM; timed from a graph
    of the 48 launches with HIP events on their stream.  The CPU baseline is
    the oracle's fused quant + GEMV over the same copies."""
    import numpy as np
    import torch
    from harsh4b_amd.lightspark import LiteSparkProjection, quant_int4_gemv
    from harsh4b_amd.synthetic import random_packed
    rows, width, copies = GEMV_ROWS, GEMV_WIDTH, GEMV_COPIES
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    w_all = random_packed(rows * copies, width, gen, dev).view(copies, rows, width // 2)
    s_all = (torch.rand((copies, rows), generator=gen, device=dev) * 0.015 + 0.005).contiguous()
    projs = [LiteSparkProjection(w_all[i], s_all[i]) for i in range(copies)]
    x = torch.from_numpy(np.random.default_rng(2).standard_normal(width).astype(np.float32)).to(dev)
    out = torch.empty(rows, dtype=torch.float32, device=dev)
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        for p in projs:
            quant_int4_gemv(x, p, out=out, stream=s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for p in projs:
            quant_int4_gemv(x, p, out=out, stream=s)
    reps = max(2, args.gemv_reps)
    with torch.cuda.stream(s):
        g.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            g.replay()
        e1.record(s)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * copies)
    nbytes = rows * width // 2 + 4 * rows + 4 * width + 4 * rows
    gbs = nbytes / (us * 1e-6) / 1e9
    result = {"workload": "configs[0]: fused quant + int4 GEMV, K=2560 -> N=9728, 48 rotating weight copies",
              "us_per_call": round(us, 3), "calls": reps * copies, "algorithmic_bytes": nbytes,
              "roofline": {"kernel": "gemv_rr_kernel (hq_quant_int4_gemv)", "bound": "hbm", "achieved": round(gbs, 1),
                           "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                           "traffic": None}}
    del g
    if cpu_seconds:
        import oracle
        hw = w_all.cpu().numpy()
        hs = s_all.cpu().numpy()
        hx = x.cpu().numpy()
        oracle.quant_int4_gemv(hx, hw[0], hs[0])

        def run(sec):
            n, t0 = 0, time.perf_counter()
            while time.perf_counter() - t0 < sec or n < 10:
                i = n % copies
                oracle.quant_int4_gemv(hx, hw[i], hs[i])
                n += 1
            el = time.perf_counter() - t0
            return n * nbytes / el / 1e9, f"{n} calls in {el:.1f} s"
        result["cpu_baseline"] = cpu_runs(run, cpu_seconds, "GB/s", "fused quant + GEMV calls over the 48 copies")
    del projs, w_all, s_all
    torch.cuda.empty_cache()
    return result


def bench_gemv(args):
    """configs[0] alone, as its own JSON line."""
    res = gemv_case(args, 0 if args.no_cpu_baseline else max(2.0, args.cpu_seconds / 2))
    gbs = res["roofline"]["achieved"]
    result = {"metric": "single fused quant + int4 GEMV (configs[0]) HBM GB/s", "value": gbs,
              "unit": "GB/s", "n_gpus": 1, "steps": res["calls"], "warmup": GEMV_COPIES,
              "us_per_call": res["us_per_call"], "higher_is_better": True, "dtype": "int8",
              "data": "synthetic", "config": {"workload": res["workload"]}, "roofline": res["roofline"]}
    if "cpu_baseline" in res:
        result["cpu_baseline"] = res["cpu_baseline"]
    print(json.dumps(result), flush=True)


def batched_step_bytes(config, m, context):
    """Algorithmic bytes of one batched decode step of m sequences at
    `context` positions each: every weight once (packed body, row scales,
    norm weights, the tied int4 LM head and its scales), each sequence's
    K/V rows (fp16, context - 1 read + 1 written per layer), its embedding
    row, RoPE rows and logits."""
    from harsh4b_amd.config import body_bytes, shapes
    L = int(config["num_hidden_layers"])
    h = int(config["hidden_size"])
    d = int(config["head_dim"])
    kvh = int(config["num_key_value_heads"])
    v = int(config["vocab_size"])
    weights = body_bytes(config) + 4 * L * sum(r for r, _ in shapes(config).values()) + 4 * L * (2 * h + 2 * d)
    lm_head = v * h // 2 + 4 * v + 4 * h
    per_seq = L * 2 * kvh * d * 2 * context + h // 2 + 4 + 4 * L * d + 4 * v
    return weights + lm_head + m * per_seq


def batched_case(model, ctx, sizes, steps, warmup, cpu_seconds, ref=None, fill=False, large_capacity=False):
    """batched greedy decode of M independent sequences (M in
    `sizes`) at context `ctx` (each prefilled with its own random ctx-token
    prompt, or with `fill` given N(0,1) K/V in its cache), one hq_decode_batch
    step per token of every sequence, replayed from a HIP graph.  Per M: the
    step time, sequence-tokens/s, the step's HBM bytes over its time (weights
    once per step + M K/V caches), and the ratio to M batch-1 decode steps of
    the same model at the same context.  The largest M gives the case's value
    and roofline.  With `large_capacity`, the smallest M is timed again with
    every state's capacity at 4096 positions."""
    import numpy as np
    import torch
    cfg = model.config
    vocab = int(cfg["vocab_size"])
    cap = ctx + warmup + steps + 4

    def prompt(i):
        return [int(t) for t in np.random.default_rng(4 + i).integers(0, vocab, ctx)]

    def start(st, i):
        if fill:
            fill_long(st, ctx, torch)
        else:
            model.prefill(prompt(i), st)

    def timed(fn):
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(model.stream)
        fn()
        e1.record(model.stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3

    # batch 1 at the same context: the rate M independent steps would have
    one = model.new_state(cap)
    start(one, 0)
    model.decode_greedy(one, warmup)
    t1 = timed(lambda: model.decode_greedy(one, steps, check_status=False))
    one.check_status()
    del one
    tok1 = steps / t1
    print(f"# configs[3] batch 1 at context {ctx}: {tok1:.1f} tok/s", file=sys.stderr, flush=True)
    per_m = {}
    for m in sizes:
        states = []
        for i in range(m):
            st = model.new_state(cap)
            start(st, i)
            states.append(st)
        model.decode_greedy_batch(states, warmup)          # captures the batched step
        t = timed(lambda: model.decode_greedy_batch(states, steps, check_status=False))
        for st in states:
            st.check_status()
        ms = t * 1e3 / steps
        nbytes = batched_step_bytes(cfg, m, ctx + warmup + steps // 2)
        gbs = nbytes / (ms * 1e-3) / 1e9
        per_m[m] = {"ms_per_step": round(ms, 3), "tok_s": round(m * steps / t, 1),
                    "speedup_vs_batch1": round(m * steps / t / tok1, 2),
                    "step_vs_batch1_step": round(ms / (1e3 / tok1), 2),
                    "achieved_GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                    "bytes_per_step": nbytes}
        print(f"# M={m}: {ms:.3f} ms/step, {m * steps / t:.1f} tok/s, {gbs:.0f} GB/s "
              f"({ms / (1e3 / tok1):.2f}x the batch-1 step)", file=sys.stderr, flush=True)
        model._batch_graph = None
        del states
    # the same M = sizes[0] with every state's capacity at 4096 positions:
    # the step's attention tails and merged qkv + attention launch cover
    # capacities of up to 512 positions (eight 64-position chunks, fixed when
    # the step's graph is captured), so a larger capacity takes the separate
    # combine, quantization and qkv kernels at any context
    big = {}
    if large_capacity:
        m = sizes[0]
        states = []
        for i in range(m):
            st = model.new_state(4096)
            start(st, i)
            states.append(st)
        model.decode_greedy_batch(states, warmup)
        t = timed(lambda: model.decode_greedy_batch(states, steps, check_status=False))
        for st in states:
            st.check_status()
        ms = t * 1e3 / steps
        big[m] = {"capacity": 4096, "ms_per_step": round(ms, 3), "tok_s": round(m * steps / t, 1),
                  "step_vs_batch1_step": round(ms / (1e3 / tok1), 2)}
        print(f"# M={m} at capacity 4096: {ms:.3f} ms/step, {m * steps / t:.1f} tok/s", file=sys.stderr,
              flush=True)
        model._batch_graph = None
        del states
    top_m = sizes[-1]
    top = per_m[top_m]
    res = {"workload": f"configs[3]: batched decode of M = {'/'.join(map(str, sizes))} sequences at context "
                       f"{ctx}, each with its own fp16 KV cache ({'N(0,1) K/V' if fill else 'prefilled prompt'}), "
                       f"greedy; value at M = {top_m}",
           "value": top["tok_s"], "unit": "sequence-tok/s", "steps": steps, "warmup": warmup,
           "ms_per_step": top["ms_per_step"],
           "roofline": {"kernel": f"whole batched step (hq_decode_batch), M={top_m}", "bound": "hbm",
                        "achieved": top["achieved_GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": top["hbm_frac"], "traffic": None, "algorithmic_bytes": top["bytes_per_step"]},
           "batch1_tok_s": round(tok1, 1), "per_m": per_m}
    if big:
        res["per_m_capacity_4096"] = big
    if cpu_seconds > 0:
        res["cpu_baseline"] = cpu_baseline_batched(model, ctx, cpu_seconds, ref)
    return res


def bench_batched(args):
    """configs[3] as its own line (see batched_case): M = --batch-sizes
    (default 8, 16, 32) at context 256; value = sequence-tokens/s at the
    largest M."""
    from harsh4b_amd.config import QWEN3_4B
    from harsh4b_amd.synthetic import random_model
    ctx = args.ctx if args.ctx is not None else 256
    steps, warmup = max(1, min(args.steps, 64)), max(1, min(args.warmup, 8))
    sizes = sorted({int(x) for x in args.batch_sizes.split(",") if x.strip()})
    if not sizes or sizes[0] < 1:
        raise SystemExit("--batch-sizes needs positive integers")
    print(f"# building random Qwen3-4B int4 model (seed {args.seed})", file=sys.stderr, flush=True)
    model = random_model(QWEN3_4B, seed=args.seed)
    case = batched_case(model, ctx, sizes, steps, warmup, 0 if args.no_cpu_baseline else args.cpu_seconds,
                        fill=args.batch_fill)
    top_m = sizes[-1]
    result = {"metric": f"batched greedy decode sequence-tokens/s (configs[3], M={top_m}, context {ctx})",
              "value": case["value"], "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
              "ms_per_step": case["ms_per_step"], "higher_is_better": True, "scaling": "weak",
              "vs_baseline": None, "dtype": "int8",
              "data": f"synthetic: random-init int4 weights, random {ctx}-token prompts (seeds 4+i)",
              "config": {"workload": case["workload"], "global_batch": top_m, "seq_len": ctx,
                         "parallelism": "none (1 GPU)"},
              "roofline": case["roofline"], "batch1_tok_s": case["batch1_tok_s"], "per_m": case["per_m"]}
    if "cpu_baseline" in case:
        result["cpu_baseline"] = case["cpu_baseline"]
    print(json.dumps(result), flush=True)


def cpu_baseline_batched(model, ctx, seconds, ref=None):
    """The oracle decoding sequences one step at a time (the reference has no
    batching: M sequences cost M steps), from a cache of `ctx` positions.
    `ref`: an oracle model of the same weights, if one is at hand."""
    import numpy as np
    import oracle
    from harsh4b_amd.synthetic import host_arrays
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    if ref is None:
        ref = oracle.OracleModel(model.config, host_arrays(model))
    rs = ref.new_state(ctx + 64)
    rng = np.random.default_rng(4)
    for name in ("keys", "values"):
        getattr(rs, name)[:, :ctx] = rng.standard_normal(getattr(rs, name)[:, :ctx].shape).astype(
            np.float16).view(np.uint16)
    rs.position = ctx
    token = ref.forward_token(1000, rs)
    n, t0 = 0, time.perf_counter()
    while True:
        token = ref.forward_token(token, rs)
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds and n >= 2) or rs.position >= rs.struct.capacity:
            break
    return {"value": round(n / el, 2), "unit": "sequence-tokens/s", "cores": threads, "kind": "port",
            "sample": f"{n} decode steps of one sequence at context {ctx}+ ({el:.1f} s; M sequences take M "
                      f"times as long), OpenMP over GEMV rows (oracle/hq_oracle.c)"}


def bench_sample(args):
    """hq_sample_token alone over Qwen3-4B's vocabulary (151936 logits, 64
    generated ids): mean time per call from HIP events over `--steps` calls,
    at the reference runner's default policy (temperature 0.7, top-k 40,
    top-p 0.9, penalty 1.08) and at other top-k."""
    import torch
    from harsh4b_amd import _native
    lib = _native.lib()
    dev = torch.device("cuda", 0)
    n = 151936
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    logits = torch.randn(n, device=dev, generator=gen) * 3
    ids = torch.randint(0, n, (64,), device=dev, dtype=torch.int32, generator=gen)
    u = torch.tensor([0.37], dtype=torch.float64, device=dev)
    out = torch.empty(1, dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream()
    per_k = {}
    for k in (40, 1, 64, 512, 2048):
        ws = torch.zeros(lib.hq_sample_workspace_bytes(n, k), dtype=torch.uint8, device=dev)

        def call():
            if lib.hq_sample_token(logits.data_ptr(), n, ids.data_ptr(), 64, 1.08, 0.7, k, 0.9, u.data_ptr(),
                                   out.data_ptr(), None, None, ws.data_ptr(), s.cuda_stream):
                raise RuntimeError("hq_sample_token failed")
        for _ in range(args.warmup):
            call()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(args.steps):
            call()
        e1.record(s)
        torch.cuda.synchronize()
        per_k[k] = e0.elapsed_time(e1) * 1e3 / args.steps
        print(f"# top_k {k:5d}: {per_k[k]:8.2f} us per token", file=sys.stderr, flush=True)
    result = {"metric": "GPU stochastic sampler tokens/s (151936 logits, reference runner's default policy)",
              "value": round(1e6 / per_k[40], 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
              "warmup": args.warmup, "ms_per_step": round(per_k[40] / 1e3, 5), "higher_is_better": True,
              "scaling": "weak", "vs_baseline": None, "dtype": "f32",
              "data": "synthetic: N(0,9) logits, 64 random generated ids",
              "config": {"workload": "hq_sample_token alone: temperature 0.7, top-k 40, top-p 0.9, penalty 1.08"},
              "us_per_token_by_top_k": {str(k): round(v, 2) for k, v in per_k.items()}}
    print(json.dumps(result), flush=True)


def bench_copy(args):
    """Calibration for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE: a plain copy
    of 256 MiB (256 MiB read + 256 MiB written per dispatch), so a counter's
    reading per dispatch divided into the known bytes gives its scale."""
    import torch
    nbytes = 256 << 20
    dev = torch.device("cuda", 0)
    src = torch.ones(nbytes // 4, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    reps = max(1, min(args.steps, 16))
    dst.copy_(src)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    gbs = 2 * nbytes / (us * 1e-6) / 1e9
    print(json.dumps({"metric": "device copy GB/s (read + write), PMC calibration", "value": round(gbs, 1),
                      "unit": "GB/s", "n_gpus": 1, "steps": reps, "warmup": 1, "bytes_read": nbytes,
                      "bytes_written": nbytes, "us_per_copy": round(us, 2), "higher_is_better": True,
                      "dtype": "int32", "data": "synthetic",
                      "config": {"workload": "copy 256 MiB"}}), flush=True)


def fill_long(state, ctx, torch):
    """the first ctx positions of every layer's cache hold N(0,1)
    keys and values (fp16); decoding starts at position ctx."""
    gen = torch.Generator(device=state.keys.device)
    gen.manual_seed(5)
    for cache in (state.keys, state.values):
        cache[:, :ctx].normal_(generator=gen)
    state.device_position.fill_(ctx)
    state.position = ctx
    state.token.fill_(1000)
    torch.cuda.synchronize()


def kv_read_bytes(config, context):
    """fp16 K/V bytes the attention of one step reads at `context` positions
    (the context - 1 cached rows of every layer)."""
    L = int(config["num_hidden_layers"])
    row = 2 * int(config["num_key_value_heads"]) * int(config["head_dim"]) * 2
    return L * row * (context - 1)


def layer_case(cfg, per_kind_ms, layers_ms, ref_arrays, cpu_seconds):
    """one decoder layer's body GEMVs at batch 1 with fused
    activation quant (and the RMSNorms in the qkv and gate_up kernels): the
    sum of the four standalone GEMV kernels (timed from graphs of each kind's
    36 launches), and the layer kernel's per-layer share (its attention and
    hand-offs included).  CPU: the oracle's fused quant + GEMV over layer 0's
    four matrices of each layer in turn (all 36, so the host's caches do not
    hold the weights)."""
    L = int(cfg["num_hidden_layers"])
    alg = algorithmic_bytes(cfg)
    nbytes = sum(alg.values())
    us = sum(per_kind_ms.values()) * 1e3
    gbs = nbytes / (us * 1e-6) / 1e9
    eng_us = layers_ms * 1e3 / L
    eng_bytes = layer_kernel_bytes(cfg, 1) // L
    res = {"workload": "configs[1]: one Qwen3-4B decoder layer's body GEMVs at batch 1 with fused quant",
           "us_per_layer": round(us, 3), "algorithmic_bytes": nbytes,
           "roofline": {"kernel": "gemv_rr_kernel x3 (qkv, o, down) + gemv_kernel (gate_up); five-kernels-per-layer form",
                        "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
           "layer_kernel_share": {"us_per_layer": round(eng_us, 3),
                                  "GB/s": round(eng_bytes / (eng_us * 1e-6) / 1e9, 1),
                                  "note": "layer kernel time / 36 (attention, norms and hand-offs included)"}}
    if cpu_seconds and ref_arrays is not None:
        import numpy as np
        import oracle
        rng = np.random.default_rng(7)
        layers = []
        for li in range(L):
            mats = []
            for name in ("qkv", "o", "gate_up", "down"):
                w, s = ref_arrays[name][li], ref_arrays[name + "_scales"][li]
                mats.append((rng.standard_normal(2 * w.shape[1]).astype(np.float32), w, s))
            layers.append(mats)

        def run(sec):
            n, t0 = 0, time.perf_counter()
            while time.perf_counter() - t0 < sec or n < 4:
                for x, w, s in layers[n % L]:
                    oracle.quant_int4_gemv(x, w, s)
                n += 1
            el = time.perf_counter() - t0
            return n * nbytes / el / 1e9, f"{n} layers in {el:.1f} s ({el / n * 1e3:.2f} ms per layer)"
        res["cpu_baseline"] = cpu_runs(run, cpu_seconds, "GB/s", "fused quant + GEMV of the four body matrices "
                                                                   f"of each of the {L} layers in turn")
    return res


def attention_case(args, torch, context=4096):
    """The standalone fused GQA decode kernel (hq_gqa_decode) at one layer's
    shape: 32 query / 8 kv heads x 128, fp16 N(0,1) K/V of `context`
    positions; timed from a graph of 36 calls (one per layer, each on its own
    cache slab, so the K/V stream from HBM and not from the last call's
    cache)."""
    from harsh4b_amd.lightspark import gqa_decode
    dev = torch.device("cuda", 0)
    L, kv, g, d = 36, 8, 4, 128
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    keys = torch.randn((L, context, kv, d), generator=gen, device=dev).half()
    values = torch.randn((L, context, kv, d), generator=gen, device=dev).half()
    q = torch.randn((kv * g * d,), generator=gen, device=dev)
    out = torch.empty_like(q)
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        for layer in range(L):
            gqa_decode(q, keys[layer], values[layer], out, context, kv, g, d, stream=s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        for layer in range(L):
            gqa_decode(q, keys[layer], values[layer], out, context, kv, g, d, stream=s)
    reps = max(2, args.gemv_reps)
    with torch.cuda.stream(s):
        graph.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            graph.replay()
        e1.record(s)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * L)
    nbytes = 2 * context * kv * d * 2 + 2 * 4 * kv * g * d
    gbs = nbytes / (us * 1e-6) / 1e9
    del graph, keys, values
    torch.cuda.empty_cache()
    return {"kernel": "attention_kernel (hq_gqa_decode)", "context": context, "us_per_call": round(us, 3),
            "algorithmic_bytes": nbytes, "achieved": round(gbs, 1), "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4)}


def bench_attention(args):
    """The standalone hq_gqa_decode at one layer's shape and context --ctx
    (default 4096) as its own JSON line (for rocprofv3 runs of that kernel
    alone)."""
    import torch
    ctx = args.ctx if args.ctx is not None else 4096
    res = attention_case(args, torch, context=ctx)
    print(json.dumps({"metric": "standalone fused GQA decode (hq_gqa_decode) HBM GB/s", "value": res["achieved"],
                      "unit": "GB/s", "n_gpus": 1, "steps": max(2, args.gemv_reps) * 36, "warmup": 36,
                      "us_per_call": res["us_per_call"], "higher_is_better": True, "dtype": "fp16/f32",
                      "data": "synthetic: N(0,1) fp16 K/V, 32 query / 8 kv heads x 128",
                      "config": {"workload": f"hq_gqa_decode at context {ctx}, 36 distinct caches"},
                      "roofline": {"kernel": res["kernel"], "bound": "hbm", "achieved": res["achieved"],
                                   "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": res["frac"], "traffic": None,
                                   "algorithmic_bytes": res["algorithmic_bytes"]}}), flush=True)


def long_case(args, model, lib, cfg, ref, cpu_seconds, short):
    """the batch-1 decode at context 4096 over an N(0,1) fp16 KV
    cache: the layer kernel at the line's context (roofline with the K/V
    bytes), the decode rate, and the attention's marginal KV bandwidth
    against the short-context launch `short` = (context, ms)."""
    import torch
    ctx, warm, steps = 4096, 16, 64
    state = model.new_state(ctx + warm + steps + 4)
    fill_long(state, ctx, torch)
    model.decode_greedy(state, warm)
    state.synchronize()
    context = int(state.device_position.item()) + 1
    layers_ms = time_layers(lib, model, state, 4, args.gemv_reps, torch)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(state.stream)
    model.decode_greedy(state, steps, check_status=False)
    e1.record(state.stream)
    torch.cuda.synchronize()
    state.check_status()
    tok_s = steps / (e0.elapsed_time(e1) / 1e3)
    eng_bytes = layer_kernel_bytes(cfg, context)
    gbs = eng_bytes / (layers_ms * 1e-3) / 1e9
    kv_extra = kv_read_bytes(cfg, context) - kv_read_bytes(cfg, short[0])
    marginal = kv_extra / ((layers_ms - short[1]) * 1e-3) / 1e9
    print(f"# configs[4]: layer kernel {layers_ms * 1e3:.1f} us at context {context}, decode {tok_s:.1f} tok/s, "
          f"attention marginal {marginal:.0f} GB/s", file=sys.stderr, flush=True)
    res = {"workload": f"configs[4]: the same decode at context {ctx} (N(0,1) fp16 KV cache), greedy",
           "tok_s": round(tok_s, 2), "steps": steps, "warmup": warm,
           "roofline": {"kernel": "engine_kernel (persistent layer kernel: 36 decoder layers)", "bound": "hbm",
                        "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic_at(context),
                        "algorithmic_bytes": eng_bytes, "context": context,
                        "us_per_launch": round(layers_ms * 1e3, 2)},
           "attention_marginal": {"kv_bytes": kv_extra, "us": round((layers_ms - short[1]) * 1e3, 2),
                                  "GB/s": round(marginal, 1), "frac": round(marginal / HBM_PEAK_GBS, 4),
                                  "note": f"extra K/V bytes read at context {context} over context {short[0]} "
                                          "/ the extra layer-kernel time"}}
    if cpu_seconds and ref is not None:
        rs = oracle_state_from(ref, state, context - 1, context + CPU_WARMUP_TOKENS + 256)
        res["cpu_baseline"] = cpu_runs(lambda sec: oracle_decode_rate(ref, rs, context - 1, sec), cpu_seconds,
                                       "tok/s", f"decode steps of the same model at context {context}, "
                                                "OpenMP over GEMV rows (oracle/hq_oracle.c)")
        del rs
    del state
    torch.cuda.empty_cache()
    return res


def layers_context(args):
    """Context of the layer-kernel launches of --workload layers: the default
    line's (a 64-token prompt and --warmup decode steps) or, for --ctx of
    1024 and more, the long workload's (an N(0,1) cache of ctx positions and
    --warmup decode steps)."""
    ctx = args.ctx if args.ctx is not None else 64
    return ctx + args.warmup + 1


def bench_layers(args):
    """The layer kernel alone, launched --steps times at the context of
    layers_context(args), for rocprofv3 --pmc (one launch = one step's 36
    decoder layers; the position does not advance between launches)."""
    import numpy as np
    import torch
    from harsh4b_amd import _native
    from harsh4b_amd.config import QWEN3_4B
    from harsh4b_amd.synthetic import random_model
    cfg = QWEN3_4B
    lib = _native.lib()
    ctx = args.ctx if args.ctx is not None else 64
    model = random_model(cfg, seed=args.seed)
    state = model.new_state(ctx + args.warmup + 8)
    if ctx >= 1024:
        fill_long(state, ctx, torch)
    else:
        model.prefill([int(t) for t in np.random.default_rng(3).integers(0, int(cfg["vocab_size"]), ctx)], state)
    model.decode_greedy(state, args.warmup)
    state.synchronize()
    context = int(state.device_position.item()) + 1
    assert context == layers_context(args), (context, layers_context(args))
    s = state.stream
    for _ in range(args.steps):
        _native.check(lib.hq_step_layers(ctypes.byref(model.struct), ctypes.byref(state.struct), s.cuda_stream),
                      "hq_step_layers")
    torch.cuda.synchronize()
    state.check_status()
    print(json.dumps({"workload": "layers", "context": context, "launches": args.steps}), flush=True)


def pmc_counter(directory, counter):
    """Mean Counter_Value per dispatch of each kernel in a rocprofv3 CSV
    output directory -> {kernel: (dispatches, mean)}."""
    import csv
    rows = {}
    for f in Path(directory).rglob("*counter_collection.csv"):
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                if r.get("Counter_Name") != counter:
                    continue
                rows.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
    return {k: (len(v), sum(v) / len(v)) for k, v in rows.items()}


def pmc_durations(directory):
    """Mean dispatch duration (ns, from the rows' timestamps) of each kernel
    in a rocprofv3 CSV output directory -> {kernel: ns}."""
    import csv
    seen = {}
    for f in Path(directory).rglob("*counter_collection.csv"):
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                seen[(r["Kernel_Name"], r["Dispatch_Id"])] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    per = {}
    for (k, _), ns in seen.items():
        per.setdefault(k, []).append(ns)
    return {k: sum(v) / len(v) for k, v in per.items()}


def pmc_summary(args):
    """HBM traffic per launch of the layer kernel from two rocprofv3 --pmc
    runs of --workload layers (FETCH_SIZE, then WRITE_SIZE; KiB per
    dispatch) scaled by what the same counters read for the 256 MiB copy of
    --workload copy."""
    from harsh4b_amd.config import QWEN3_4B
    fetch_dir, write_dir, cfetch_dir, cwrite_dir = args.pmc_summary
    copy_bytes = 256 << 20

    def copy_kib(d, counter):
        for k, (_, v) in pmc_counter(d, counter).items():
            if "copyBuffer" in k or "copy" in k.lower():
                return v
        raise SystemExit(f"no copy kernel in {d}")
    cf, cw = copy_kib(cfetch_dir, "FETCH_SIZE"), copy_kib(cwrite_dir, "WRITE_SIZE")
    ff, wf = copy_bytes / (cf * 1024), copy_bytes / (cw * 1024)
    fetch, write = pmc_counter(fetch_dir, "FETCH_SIZE"), pmc_counter(write_dir, "WRITE_SIZE")
    name = next(k for k in fetch if "engine_kernel" in k)
    n, fk = fetch[name]
    wk = write[name][1]
    context = layers_context(args)
    traffic = int(fk * 1024 * ff + wk * 1024 * wf)
    alg = layer_kernel_bytes(QWEN3_4B, context)
    print(json.dumps({"calibration": {"copy_kernel_bytes_read": copy_bytes, "copy_kernel_bytes_written": copy_bytes,
                                      "copy_fetch_kib": round(cf, 1), "copy_write_kib": round(cw, 1),
                                      "fetch_factor": round(ff, 4), "write_factor": round(wf, 4)},
                      "runs": [{"kernel": name, "context": context, "dispatches": n, "fetch_kib": round(fk, 1),
                                "write_kib": round(wk, 1), "traffic_bytes": traffic, "algorithmic_bytes": alg,
                                "ratio": round(traffic / alg, 4)}]}, indent=1), flush=True)


MI355X_CLOCK_GHZ = 2.4   # peak engine clock: MFMA utilisation against it is a lower bound


def pmc_kernels(args):
    """Per-kernel counters of one workload from rocprofv3 --pmc runs: MFMA
    utilisation (SQ_VALU_MFMA_BUSY_CYCLES, summed over the SIMDs, / (the
    dispatch's duration x the 2.4 GHz peak clock x 1024 SIMDs)), int8 MFMA
    ops per dispatch (SQ_INSTS_VALU_MFMA_MOPS_I8 x 512) and per second of the
    dispatch, and HBM bytes per dispatch (FETCH_SIZE, WRITE_SIZE scaled by a
    256 MiB copy's readings).  Durations are those of the counter runs
    (dispatches serialized by the profiler)."""
    mfma_dir, fetch_dir, write_dir, cfetch_dir, cwrite_dir = args.pmc_kernels
    copy_bytes = 256 << 20

    def copy_kib(d, counter):
        for k, (_, v) in pmc_counter(d, counter).items():
            if "copyBuffer" in k or "copy" in k.lower():
                return v
        raise SystemExit(f"no copy kernel in {d}")
    ff = copy_bytes / (copy_kib(cfetch_dir, "FETCH_SIZE") * 1024)
    wf = copy_bytes / (copy_kib(cwrite_dir, "WRITE_SIZE") * 1024)
    mops = pmc_counter(mfma_dir, "SQ_INSTS_VALU_MFMA_MOPS_I8")
    busy = pmc_counter(mfma_dir, "SQ_VALU_MFMA_BUSY_CYCLES")
    dur = pmc_durations(mfma_dir)
    fetch, write = pmc_counter(fetch_dir, "FETCH_SIZE"), pmc_counter(write_dir, "WRITE_SIZE")
    simds = 256 * 4
    rows = []
    for k in sorted(mops, key=lambda n: -mops[n][0] * dur.get(n, 0.0)):
        n = mops[k][0]
        ns = dur.get(k, 0.0)
        r = {"kernel": k[:120], "dispatches": n, "us": round(ns / 1e3, 2), "int8_ops": round(mops[k][1] * 512)}
        if ns > 0:
            r["int8_TOPS"] = round(mops[k][1] * 512 / ns / 1e3, 2)
            if k in busy:
                r["mfma_util"] = round(busy[k][1] / (ns * MI355X_CLOCK_GHZ * simds), 5)
        if k in fetch:
            r["hbm_read_bytes"] = round(fetch[k][1] * 1024 * ff)
        if k in write:
            r["hbm_write_bytes"] = round(write[k][1] * 1024 * wf)
        if ns > 0 and "hbm_read_bytes" in r and "hbm_write_bytes" in r:
            r["hbm_GBs"] = round((r["hbm_read_bytes"] + r["hbm_write_bytes"]) / ns, 1)
        rows.append(r)
    print(json.dumps({"calibration": {"fetch_factor": round(ff, 4), "write_factor": round(wf, 4)},
                      "kernels": rows[:24]}, indent=1), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the path runs on one GPU's share; sharding across GPUs is not built)", file=sys.stderr)
        sys.exit(2)
    if args.pmc_summary:
        pmc_summary(args)
        return
    if args.pmc_kernels:
        pmc_kernels(args)
        return
    if args.workload == "layers":
        bench_layers(args)
        return
    if args.workload == "gemv":
        bench_gemv(args)
        return
    if args.workload == "copy":
        bench_copy(args)
        return
    if args.workload == "sample":
        bench_sample(args)
        return
    if args.workload == "batched":
        bench_batched(args)
        return
    if args.workload == "attention":
        bench_attention(args)
        return
    import numpy as np
    import torch
    from harsh4b_amd import _native
    from harsh4b_amd.config import QWEN3_4B, body_bytes
    from harsh4b_amd.synthetic import random_model

    cfg = QWEN3_4B
    lib = _native.lib()
    long_ctx = args.workload == "long"
    if args.ctx is None:
        args.ctx = 4096 if long_ctx else 64
    print(f"# building random Qwen3-4B int4 model (seed {args.seed})", file=sys.stderr, flush=True)
    model = random_model(cfg, seed=args.seed)
    cap = args.ctx + args.warmup + args.steps + 4
    state = model.new_state(cap)
    if long_ctx:
        fill_long(state, args.ctx, torch)
        print(f"# filled {args.ctx} cache positions with N(0,1)", file=sys.stderr, flush=True)
    else:
        prompt = [int(t) for t in np.random.default_rng(3).integers(0, int(cfg["vocab_size"]), args.ctx)]
        # the prompt through the batched prefill, and the same prompt token
        # by token on a second state (the reference's loop), both timed
        scratch = model.new_state(cap)
        model.prefill(prompt[:2], scratch)          # first-use allocations and code loads
        scratch.synchronize()
        del scratch
        t0 = time.perf_counter()
        model.prefill(prompt, state)
        state.synchronize()
        prefill_s = time.perf_counter() - t0
        loop_state = model.new_state(cap)
        t0 = time.perf_counter()
        for t in prompt:
            model.forward_token(t, loop_state)
        loop_state.synchronize()
        loop_s = time.perf_counter() - t0
        del loop_state
        prefill_info = {"tokens": args.ctx, "ms_batched": round(prefill_s * 1e3, 2),
                        "ms_token_loop": round(loop_s * 1e3, 2),
                        "note": "wall time to logits of the last prompt token, one run each"}
        print(f"# prefilled {args.ctx} tokens: batched {prefill_s * 1e3:.1f} ms, token loop "
              f"{loop_s * 1e3:.1f} ms", file=sys.stderr, flush=True)

    if long_ctx:
        prefill_info = None
    policy = generator = None
    if args.workload == "sampled":
        from types import SimpleNamespace
        from harsh4b_amd.lightspark import sample_logits
        policy = SimpleNamespace(argmax=False, temperature=0.7, top_k=40, top_p=0.9, repetition_penalty=1.08)
        generator = np.random.default_rng(args.seed)
        generated = [sample_logits(state.logits, [], policy, generator)]
        generated += model.decode_sampled(state, args.warmup, policy, generator, generated)
    else:
        model.decode_greedy(state, args.warmup)      # captures the step graph
    state.synchronize()
    # The dominant kernel, measured live: the persistent layer kernel (all
    # 36 decoder layers of a step, ~96 % of the step time), replayed from a
    # graph at the first decode position (its K/V row there is rewritten by
    # the decode step that follows).
    L = int(cfg["num_hidden_layers"])
    context = int(state.device_position.item()) + 1
    layers_ms = time_layers(lib, model, state, 4, args.gemv_reps, torch)
    eng_bytes = layer_kernel_bytes(cfg, context)
    achieved = eng_bytes / (layers_ms * 1e-3) / 1e9
    body_gbs = body_bytes(cfg) / (layers_ms * 1e-3) / 1e9
    print(f"# layer kernel: {layers_ms * 1e3:.1f} us/launch at context {context}, "
          f"{achieved:.1f} GB/s ({body_gbs:.1f} GB/s of body weights)", file=sys.stderr, flush=True)

    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(state.stream)
    if policy is not None:
        generated += model.decode_sampled(state, args.steps, policy, generator, generated)
    else:
        model.decode_greedy(state, args.steps, check_status=False)
    e1.record(state.stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    state.check_status()
    tok_s = args.steps / (ms / 1e3)
    print(f"# decode: {args.steps} steps in {ms:.2f} ms -> {tok_s:.1f} tok/s", file=sys.stderr, flush=True)

    # The five-kernels-per-layer form of the same step (the fallback path),
    # its GEMVs timed alone: graphs of each kind's 36 launches.
    kinds = {"qkv": 0, "o": 1, "gate_up": 2, "down": 3}
    per_kind_ms = {}
    for name, kind in kinds.items():
        per_kind_ms[name] = time_graph(lib, model, state, [(l, kind) for l in range(L)],
                                       args.gemv_reps, torch) / L
    state.check_status()
    alg = algorithmic_bytes(cfg)
    for k in kinds:
        print(f"# {k:8s} GEMV kernel alone: {per_kind_ms[k] * 1e3:8.2f} us/launch, "
              f"{alg[k] / (per_kind_ms[k] * 1e-3) / 1e9:8.1f} GB/s", file=sys.stderr, flush=True)

    result = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": (None if long_ctx else
                        round(tok_s / (PUBLISHED_SAMPLED_TOK_S if policy else PUBLISHED_GREEDY_TOK_S), 2)),
        "dtype": "int8",
        "data": "synthetic: random-init int4 weights, random prompt token ids",
        "config": {"workload": (f"configs[4]: 36-layer Qwen3-4B-shaped int4 decode, batch 1, context "
                                f"{args.ctx} (N(0,1) fp16 KV cache), greedy" if long_ctx else
                                "configs[2]: 36-layer Qwen3-4B-shaped int4 decode, batch 1, "
                                f"context {args.ctx}, fp16 KV cache, " +
                                ("stochastic sampler on the GPU (temperature 0.7, top-k 40, top-p 0.9, "
                                 f"repetition penalty 1.08, seed {args.seed})" if policy else "greedy")),
                   "global_batch": 1, "seq_len": args.ctx, "parallelism": "none (1 GPU)"},
        "roofline": {"kernel": "engine_kernel (persistent layer kernel: 36 decoder layers)", "bound": "hbm",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_at(context),
                     "algorithmic_bytes": eng_bytes, "context": context,
                     "us_per_launch": round(layers_ms * 1e3, 2)},
        "body_gemv": body_gemv_metric(cfg, per_kind_ms, layers_ms),
        "per_layer_kernels": {k: {"us_per_launch": round(per_kind_ms[k] * 1e3, 3),
                                  "GB/s": round(alg[k] / (per_kind_ms[k] * 1e-3) / 1e9, 1)}
                              for k in kinds},
    }
    if prefill_info:
        result["prefill"] = prefill_info
    if args.workload == "decode" and not args.no_configs:
        result["sampled"] = sampled_case(model, prompt, args.steps, args.warmup, args.seed)
        print(f"# sampled decode: {result['sampled']['tok_s']} tok/s", file=sys.stderr, flush=True)
    ref = arrays = None
    if not args.no_cpu_baseline:
        import oracle
        from harsh4b_amd.synthetic import host_arrays
        arrays = host_arrays(model)
        ref = oracle.OracleModel(model.config, arrays)
    cpu_s = 0 if args.no_cpu_baseline else args.cpu_seconds
    if args.workload == "decode" and not args.no_configs:
        print("# configs[0], [1], [4] and [3]", file=sys.stderr, flush=True)
        configs = {"configs[0]": gemv_case(args, cpu_s / 4),
                   "configs[1]": layer_case(cfg, per_kind_ms, layers_ms, arrays, cpu_s / 4),
                   "configs[4]": long_case(args, model, lib, cfg, ref, cpu_s, (context, layers_ms))}
        print("# configs[3]", file=sys.stderr, flush=True)
        configs["configs[3]"] = batched_case(model, 256, [8, 16, 32], 16, 2, cpu_s / 4, ref, large_capacity=True)
        result["configs"] = configs
        att = attention_case(args, torch)
        print(f"# hq_gqa_decode at context 4096: {att['us_per_call']:.2f} us, {att['achieved']:.0f} GB/s",
              file=sys.stderr, flush=True)
        result["attention"] = {"standalone_ctx4096": att,
                               "layer_kernel_marginal_ctx4096": configs["configs[4]"]["attention_marginal"]}
    if ref is not None:
        print("# timing the CPU oracle baseline", file=sys.stderr, flush=True)
        # room for the warm-up and about 2000 timed tokens: the sample is
        # bounded by --cpu-seconds, not by the state
        rs = oracle_state_from(ref, state, args.ctx, args.ctx + CPU_WARMUP_TOKENS + 2048)
        result["cpu_baseline"] = cpu_baseline(ref, rs, args.ctx, cpu_s)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
