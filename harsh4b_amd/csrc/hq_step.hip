// hq_step.hip - one decode step of a Qwen3-shaped model on gfx950, plus the
// library's status helpers and HIP-graph capture of whole steps.
//
// The launch sequence follows LiteSparkQwen.forward_token
// (cpu_lightspark.py:424-468 in the reference repository).  The decoder
// layers run either as one persistent kernel (hq_engine.hip) or as five
// kernels per layer, with the same arithmetic:
//   1. RMSNorm(input) -> int8 quant -> qkv GEMV              (:431-434)
//   2. qk-norm -> RoPE -> fp16 KV write -> GQA attention     (:435-441)
//   3. int8 quant -> o GEMV -> residual add                  (:442-445)
//   4. RMSNorm(post) -> quant -> gate_up GEMV -> SwiGLU      (:447-455)
//   5. int8 quant -> down GEMV -> residual add               (:456-459)
// preceded by the embedding row decode (:429; inside the persistent
// kernel's first layer when that runs, else its own kernel) and followed by
// the final
// RMSNorm -> quant -> tied LM head GEMV -> argmax (:461-466, :704-705),
// whose last block also writes the greedy token and advances the position.
// Token and position live in device memory, so a captured graph of this
// sequence is valid at every position.
#include "hq_device.h"
#include "hq_internal.h"

namespace hq {

__global__ __launch_bounds__(kBlock) void embedding_kernel(
    const uint8_t* emb, const float* emb_scales, int vocab, int hidden, const int32_t* token,
    int32_t* status, float* x)
{
    int t = *token;
    if (t < 0 || t >= vocab) {
        if (threadIdx.x == 0) atomicOr(status, HQ_STEP_BAD_TOKEN);
        t = 0;
    }
    const int half = hidden >> 1;
    const uint8_t* row = emb + size_t(t) * size_t(half);
    const float s = emb_scales[t];
    for (int j = threadIdx.x; j < half; j += kBlock) {
        const uint8_t b = row[j];
        const int lo = int(int8_t(uint8_t(b << 4))) >> 4;
        const int hi = int(int8_t(b)) >> 4;
        x[2 * j] = float(lo) * s;
        x[2 * j + 1] = float(hi) * s;
    }
}

struct StepLayout {
    int q_size, kv_size, groups, max_chunks, lm_blocks;
    size_t attn_part_bytes, lm_val_off, lm_idx_off, lm_counter_off;
    size_t epoch_off, ll_off, eng_part_off, trace_off, total;
};

static size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

static StepLayout step_layout(const hq_model* m, int capacity)
{
    StepLayout L{};
    L.q_size = m->heads * m->head_dim;
    L.kv_size = m->kv_heads * m->head_dim;
    L.groups = m->heads / m->kv_heads;
    L.max_chunks = (capacity + kAttnChunk - 1) / kAttnChunk;
    L.lm_blocks = step_gemv_blocks(StepGemv::LmHead, m->vocab, 0, m->hidden);
    L.attn_part_bytes = align256(attention_workspace_floats(m->heads, L.max_chunks, m->head_dim) * 4);
    L.lm_val_off = L.attn_part_bytes;
    L.lm_idx_off = L.lm_val_off + align256(size_t(L.lm_blocks) * 4);
    L.lm_counter_off = L.lm_idx_off + align256(size_t(L.lm_blocks) * 4);
    L.epoch_off = L.lm_counter_off + align256(size_t(ticket_words(L.lm_blocks)) * 4);
    L.ll_off = L.epoch_off + 256;
    L.eng_part_off = L.ll_off + align256(engine_handoff_bytes(m));
    L.trace_off = L.eng_part_off + align256(size_t(m->heads) * L.max_chunks * (m->head_dim + 2) * 8);
    L.total = L.trace_off + engine_trace_bytes(m);
    return L;
}

static bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

static int validate(const hq_model* m, const hq_state* st)
{
    if (!m || !st || !m->layer) return HQ_ERR_ARG;
    if (m->layers <= 0 || m->hidden <= 0 || m->intermediate <= 0 || m->heads <= 0 ||
        m->kv_heads <= 0 || m->vocab <= 0)
        return HQ_ERR_ARG;
    if (m->head_dim != 128 || m->heads % m->kv_heads || m->heads / m->kv_heads > 4) return HQ_ERR_ARG;
    const int q = m->heads * m->head_dim;
    if ((m->hidden & 31) || (m->intermediate & 31) || (q & 31)) return HQ_ERR_ARG;
    if (m->hidden > 10240 || m->intermediate > 10240 || q > 10240) return HQ_ERR_ARG;
    if (st->capacity <= 0 || m->rope_positions < st->capacity) return HQ_ERR_ARG;
    if (!m->embedding || !m->embedding_scales || !m->final_norm || !m->rope_cos || !m->rope_sin)
        return HQ_ERR_ARG;
    if (!st->keys || !st->values || !st->position || !st->token || !st->status || !st->x ||
        !st->qkv || !st->attended || !st->activated || !st->logits || !st->workspace)
        return HQ_ERR_ARG;
    if (!a16(m->embedding) || !a16(st->workspace)) return HQ_ERR_ALIGN;
    if (m->device_layer && !a16(m->device_layer)) return HQ_ERR_ALIGN;
    for (int l = 0; l < m->layers; ++l) {
        const hq_layer& L = m->layer[l];
        if (!L.qkv || !L.o || !L.gate_up || !L.down || !L.qkv_scales || !L.o_scales ||
            !L.gate_up_scales || !L.down_scales || !L.input_norm || !L.post_norm || !L.q_norm ||
            !L.k_norm)
            return HQ_ERR_ARG;
        if (!a16(L.qkv) || !a16(L.o) || !a16(L.gate_up) || !a16(L.down)) return HQ_ERR_ALIGN;
    }
    return HQ_OK;
}

static hipError_t layer_gemv(const hq_model* m, const hq_state* st, int l, StepGemv kind,
                             hipStream_t s)
{
    const hq_layer& L = m->layer[l];
    const int H = m->hidden, I = m->intermediate;
    const int q = m->heads * m->head_dim, kv = m->kv_heads * m->head_dim;
    GemvParams p{};
    switch (kind) {
    case StepGemv::Qkv:
        p.w = L.qkv; p.ws = L.qkv_scales; p.rows = q + 2 * kv; p.width = H;
        p.xf = st->x; p.gamma = L.input_norm; p.eps = m->eps; p.out = st->qkv;
        break;
    case StepGemv::OResidual:
        p.w = L.o; p.ws = L.o_scales; p.rows = H; p.width = q;
        p.xf = st->attended; p.out = st->x;
        break;
    case StepGemv::GateUpSwiglu:
        p.w = L.gate_up; p.ws = L.gate_up_scales; p.rows = 2 * I; p.half_rows = I; p.width = H;
        p.xf = st->x; p.gamma = L.post_norm; p.eps = m->eps; p.out = st->activated;
        break;
    case StepGemv::DownResidual:
        p.w = L.down; p.ws = L.down_scales; p.rows = H; p.width = I;
        p.xf = st->activated; p.out = st->x;
        break;
    default:
        return hipErrorInvalidValue;
    }
    return launch_step_gemv(kind, p, s);
}

// The decoder layers of a step: the persistent layer kernel when the model
// carries a device layer table and fits its limits, else five kernels per
// layer.
static bool engine_runs(const hq_model* m)
{
    return m->device_layer && !(m->flags & HQ_MODEL_PER_LAYER_KERNELS) && engine_fits(m) && engine_blocks(m) > 0;
}

// embed: the layer kernel takes layer 0's input from the embedding row of
// the state's token (only when it runs; the per-layer kernels read st->x).
static hipError_t enqueue_layers(const hq_model* m, const hq_state* st, bool embed, hipStream_t s)
{
    const StepLayout Ly = step_layout(m, st->capacity);
    char* ws = static_cast<char*>(st->workspace);
    const size_t kv_layer = size_t(st->capacity) * size_t(Ly.kv_size);
    hipError_t e = hipSuccess;
    const int nb = engine_runs(m) ? engine_blocks(m) : 0;
    if (nb > 0) {
        e = launch_engine(m, st, reinterpret_cast<uint32_t*>(ws + Ly.ll_off),
                          reinterpret_cast<uint32_t*>(ws + Ly.epoch_off),
                          reinterpret_cast<uint64_t*>(ws + Ly.eng_part_off), Ly.max_chunks, nb,
                          engine_trace_bytes(m) ? reinterpret_cast<uint32_t*>(ws + Ly.trace_off) : nullptr, embed,
                          s);
        if (e != hipSuccess) return e;
    }
    for (int l = 0; nb == 0 && l < m->layers; ++l) {
        const hq_layer& L = m->layer[l];
        if ((e = layer_gemv(m, st, l, StepGemv::Qkv, s)) != hipSuccess) return e;

        AttnParams a{};
        a.qkv = st->qkv; a.q_norm = L.q_norm; a.k_norm = L.k_norm;
        a.rope_cos = m->rope_cos; a.rope_sin = m->rope_sin; a.eps = m->eps;
        a.keys = st->keys + size_t(l) * kv_layer;
        a.values = st->values + size_t(l) * kv_layer;
        a.time_stride = Ly.kv_size;
        a.position = st->position; a.capacity = st->capacity; a.status = st->status;
        a.kv_heads = m->kv_heads; a.groups = Ly.groups; a.head_dim = m->head_dim;
        a.max_chunks = Ly.max_chunks;
        a.part = reinterpret_cast<float*>(ws);
        a.out = st->attended;
        if ((e = launch_attention(a, true, s)) != hipSuccess) return e;

        if ((e = layer_gemv(m, st, l, StepGemv::OResidual, s)) != hipSuccess) return e;
        if ((e = layer_gemv(m, st, l, StepGemv::GateUpSwiglu, s)) != hipSuccess) return e;
        if ((e = layer_gemv(m, st, l, StepGemv::DownResidual, s)) != hipSuccess) return e;
    }
    return hipSuccess;
}

static hipError_t enqueue_step(const hq_model* m, const hq_state* st, hipStream_t s)
{
    const StepLayout Ly = step_layout(m, st->capacity);
    char* ws = static_cast<char*>(st->workspace);
    const int H = m->hidden;

    // the embedding lookup: folded into the layer kernel when that runs
    // (one launch and its gap fewer per token: 1244 -> 1252 tok/s at
    // context 64), else its own kernel
    const bool fold = engine_runs(m);
    if (!fold) hipLaunchKernelGGL(embedding_kernel, dim3(1), dim3(kBlock), 0, s, m->embedding,
                                  m->embedding_scales, m->vocab, H, st->token, st->status, st->x);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if ((e = enqueue_layers(m, st, fold, s)) != hipSuccess) return e;

    GemvParams p{};
    p.w = m->embedding; p.ws = m->embedding_scales; p.rows = m->vocab; p.width = H;
    p.xf = st->x; p.gamma = m->final_norm; p.eps = m->eps; p.out = st->logits;
    p.part_val = reinterpret_cast<float*>(ws + Ly.lm_val_off);
    p.part_idx = reinterpret_cast<int32_t*>(ws + Ly.lm_idx_off);
    p.counter = reinterpret_cast<int32_t*>(ws + Ly.lm_counter_off);
    p.token = st->token; p.position = st->position;
    return launch_step_gemv(StepGemv::LmHead, p, s);
}

}  // namespace hq

using namespace hq;

extern "C" const char* hq_status_string(int status)
{
    switch (status) {
    case HQ_OK: return "ok";
    case HQ_ERR_ARG: return "invalid argument (shape, size or null pointer)";
    case HQ_ERR_ALIGN: return "pointer or row alignment not met";
    case HQ_ERR_LAUNCH: return "HIP kernel launch failed";
    case HQ_ERR_DEVICE: return "no usable gfx950 device";
    default: return "unknown status";
    }
}

extern "C" int hq_abi_version(void) { return 101; }

extern "C" size_t hq_step_workspace_bytes(const hq_model* model, int capacity)
{
    if (!model || capacity <= 0 || model->head_dim <= 0 || model->kv_heads <= 0) return 0;
    return step_layout(model, capacity).total;
}

extern "C" int hq_step_layer_blocks(const hq_model* model)
{
    if (!model || !model->device_layer || (model->flags & HQ_MODEL_PER_LAYER_KERNELS) ||
        model->kv_heads <= 0 || model->heads <= 0 || !engine_fits(model))
        return 0;
    return engine_blocks(model);
}

extern "C" int hq_decode_step(const hq_model* model, const hq_state* state, void* stream)
{
    const int rc = validate(model, state);
    if (rc != HQ_OK) return rc;
    return enqueue_step(model, state, static_cast<hipStream_t>(stream)) == hipSuccess
               ? HQ_OK : HQ_ERR_LAUNCH;
}

extern "C" int hq_step_gemv(const hq_model* model, const hq_state* state, int layer, int kind,
                            void* stream)
{
    const int rc = validate(model, state);
    if (rc != HQ_OK) return rc;
    if (layer < 0 || layer >= model->layers || kind < 0 || kind > 3) return HQ_ERR_ARG;
    const StepGemv kinds[4] = {StepGemv::Qkv, StepGemv::OResidual, StepGemv::GateUpSwiglu,
                               StepGemv::DownResidual};
    return layer_gemv(model, state, layer, kinds[kind], static_cast<hipStream_t>(stream)) == hipSuccess
               ? HQ_OK : HQ_ERR_LAUNCH;
}

extern "C" int hq_step_layers(const hq_model* model, const hq_state* state, void* stream)
{
    const int rc = validate(model, state);
    if (rc != HQ_OK) return rc;
    return enqueue_layers(model, state, false, static_cast<hipStream_t>(stream)) == hipSuccess
               ? HQ_OK : HQ_ERR_LAUNCH;
}

extern "C" int hq_graph_capture(const hq_model* model, const hq_state* state, int steps,
                                void* stream, void** graph_exec)
{
    if (!graph_exec || steps <= 0 || !stream) return HQ_ERR_ARG;
    const int rc = validate(model, state);
    if (rc != HQ_OK) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) return HQ_ERR_LAUNCH;
    hipError_t e = hipSuccess;
    for (int i = 0; i < steps && e == hipSuccess; ++i) e = enqueue_step(model, state, s);
    hipGraph_t graph = nullptr;
    const hipError_t ec = hipStreamEndCapture(s, &graph);
    if (e != hipSuccess || ec != hipSuccess || !graph) {
        if (graph) (void)hipGraphDestroy(graph);
        return HQ_ERR_LAUNCH;
    }
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return HQ_ERR_LAUNCH;
    *graph_exec = exec;
    return HQ_OK;
}

extern "C" int hq_graph_launch(void* graph_exec, void* stream)
{
    if (!graph_exec) return HQ_ERR_ARG;
    return hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec),
                          static_cast<hipStream_t>(stream)) == hipSuccess ? HQ_OK : HQ_ERR_LAUNCH;
}

extern "C" int hq_graph_destroy(void* graph_exec)
{
    if (!graph_exec) return HQ_ERR_ARG;
    return hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)) == hipSuccess
               ? HQ_OK : HQ_ERR_LAUNCH;
}
