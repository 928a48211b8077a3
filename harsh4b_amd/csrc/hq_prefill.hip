// hq_prefill.hip - batched prefill: the decoder layers of a run of prompt
// tokens, processed layer by layer for the whole run, with the same
// arithmetic as the token-by-token step (LiteSparkQwen.forward_token,
// cpu_lightspark.py:424-468 in the reference repository; the reference
// prefills one token at a time, :809-810).  It writes the run's K/V rows and
// advances the position; it computes no logits (the caller forwards the
// prompt's last token with hq_decode_step for those).
//
// Per layer, for a batch of up to kPrefillBatch tokens:
//   rows<NORM | RESID_NORM>  x (+= previous down output), RMSNorm, int8 quant
//   gemm_run                 qkv for every token (int8 MFMA, = the GEMV bits)
//   prefill_qk_kernel        q/k head norm + RoPE, K/V rows -> fp16 cache
//   attention (PLAIN batch)  query z attends start + z + 1 positions
//   rows<PLAIN>, gemm_run    o
//   rows<RESID_NORM>, gemm   x += o, RMSNorm, gate_up
//   rows<SWIGLU>, gemm_run   SwiGLU, down
// Each row kernel restates the decode path's prologue for one token per
// block (256-lane fmaf partials, tree sum, quantize with the spec rounding)
// and writes the int8 row de-interleaved, as the GEMM reads it.
#include <algorithm>

#include "hq_device.h"
#include "hq_internal.h"

namespace hq {

constexpr int kPrefillBatch = 128;      // tokens per pass over the layers
constexpr int kPrefillMaxWidth = 10240; // intermediate size the SwiGLU row kernel holds in LDS

enum RowMode { ROW_NORM = 0, ROW_RESID_NORM = 1, ROW_PLAIN = 2, ROW_SWIGLU = 3 };

// Byte of column i in a de-interleaved row (per 8 columns: evens, then odds).
__device__ __forceinline__ int deint_offset(int i)
{
    return (i & ~7) + ((i & 1) ? 4 + ((i & 7) >> 1) : ((i & 7) >> 1));
}

__global__ __launch_bounds__(kBlock) void prefill_embed_kernel(const uint8_t* emb, const float* emb_scales,
                                                               int vocab, int hidden, const int32_t* tokens,
                                                               int32_t* status, float* x)
{
    int t = tokens[blockIdx.x];
    if (t < 0 || t >= vocab) {
        if (threadIdx.x == 0) atomicOr(status, HQ_STEP_BAD_TOKEN);
        t = 0;
    }
    const int half = hidden >> 1;
    const uint8_t* row = emb + size_t(t) * size_t(half);
    const float s = emb_scales[t];
    float* xr = x + size_t(blockIdx.x) * hidden;
    for (int j = threadIdx.x; j < half; j += kBlock) {
        const uint8_t b = row[j];
        const int lo = int(int8_t(uint8_t(b << 4))) >> 4;
        const int hi = int(int8_t(b)) >> 4;
        xr[2 * j] = float(lo) * s;
        xr[2 * j + 1] = float(hi) * s;
    }
}

struct RowParams {
    float* x;               // [batch, k] (NORM, RESID_NORM: the residual stream; PLAIN: the input rows)
    const float* add;       // RESID_NORM: [batch, k] added to x first (x is updated)
    const float* gate_up;   // SWIGLU: [batch, 2k] gate then up
    const float* gamma;     // NORM, RESID_NORM: [k]
    float eps;
    int k, kp;              // width; row stride of q (gemm_padded_k(k))
    int8_t* q;              // [*, kp] de-interleaved
    float* act;             // [batch]
};

template <int MODE>
__device__ __forceinline__ float row_value(const RowParams& p, int m, int i, float r)
{
    if constexpr (MODE == ROW_SWIGLU) {
        const float g = p.gate_up[size_t(m) * 2 * p.k + i];
        const float u = p.gate_up[size_t(m) * 2 * p.k + p.k + i];
        const float t = 1.0f + spec_expf(-g);
        return (g / t) * u;
    } else if constexpr (MODE == ROW_PLAIN) {
        return p.x[size_t(m) * p.k + i];
    } else {
        return (p.x[size_t(m) * p.k + i] / r) * p.gamma[i];
    }
}

// One token (block) per row: the prologue of the step's GEMVs.
template <int MODE>
__global__ __launch_bounds__(kBlock) void prefill_rows_kernel(RowParams p)
{
    __shared__ float red[kBlock];
    const int m = blockIdx.x;
    const int tid = threadIdx.x;
    float r = 1.0f;
    if constexpr (MODE == ROW_NORM || MODE == ROW_RESID_NORM) {
        float* xr = p.x + size_t(m) * p.k;
        float ss = 0.0f;
        for (int i = tid; i < p.k; i += kBlock) {
            float v = xr[i];
            if constexpr (MODE == ROW_RESID_NORM) {
                v = v + p.add[size_t(m) * p.k + i];
                xr[i] = v;
            }
            ss = __builtin_fmaf(v, v, ss);
        }
        const float total = block_tree_sum256(ss, red);
        r = __builtin_sqrtf(total / float(p.k) + p.eps);
    }
    int8_t* qr = p.q + size_t(m) * p.kp;
    float amax = 0.0f;
    if constexpr (MODE == ROW_SWIGLU) {
        // the SwiGLU values (one exp each) are kept in LDS for the quant pass
        __shared__ float vals[kPrefillMaxWidth];
        for (int i = tid; i < p.k; i += kBlock) {
            const float v = row_value<MODE>(p, m, i, r);
            vals[i] = v;
            amax = fmaxf(amax, fabsf(v));
        }
        amax = block_max_nonneg(amax, red);
        amax = fmaxf(amax, 1e-5f);
        const float inv = 127.0f / amax;
        for (int i = tid; i < p.k; i += kBlock) qr[deint_offset(i)] = quant_i8(vals[i], inv);
    } else {
        for (int i = tid; i < p.k; i += kBlock) amax = fmaxf(amax, fabsf(row_value<MODE>(p, m, i, r)));
        amax = block_max_nonneg(amax, red);
        amax = fmaxf(amax, 1e-5f);
        const float inv = 127.0f / amax;
        for (int i = tid; i < p.k; i += kBlock) qr[deint_offset(i)] = quant_i8(row_value<MODE>(p, m, i, r), inv);
    }
    if (tid == 0) p.act[m] = amax / 127.0f;
}

struct QkParams {
    const float* qkv;       // [batch, (heads + 2 kv) * D]
    const float* q_norm;
    const float* k_norm;
    const float* rope_cos;  // [positions, D/2]
    const float* rope_sin;
    float eps;
    int heads, kv_heads, start;
    long long time_stride;
    uint16_t* keys;         // this layer's cache
    uint16_t* values;
    float* q;               // [batch, heads * D]
};

// Wave w of block (m, b) handles head slot 4b + w of token m: query heads
// (normed, rotated, kept fp32), then key heads (normed, rotated, stored
// fp16 at position start + m), then value heads (stored fp16).  The same
// arithmetic as the step's attention prologue (D = 128: lane holds dims
// lane and lane + 64).
__global__ __launch_bounds__(kBlock) void prefill_qk_kernel(QkParams p)
{
    constexpr int D = 128;
    const int m = blockIdx.x;
    const int slot = blockIdx.y * (kBlock / kWave) + threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const int total = p.heads + 2 * p.kv_heads;
    if (slot >= total) return;
    const int pos = p.start + m;
    const float* src = p.qkv + size_t(m) * total * D + size_t(slot) * D;
    const float x0 = src[lane], x1 = src[lane + 64];
    if (slot >= p.heads + p.kv_heads) {
        uint16_t* vdst = p.values + size_t(pos) * p.time_stride + size_t(slot - p.heads - p.kv_heads) * D;
        vdst[lane] = f32_to_f16(x0);
        vdst[lane + 64] = f32_to_f16(x1);
        return;
    }
    const bool is_q = slot < p.heads;
    const float* w = is_q ? p.q_norm : p.k_norm;
    float s = __builtin_fmaf(x0, x0, 0.0f);
    s = __builtin_fmaf(x1, x1, s);
    const float ss = wave_tree_sum64_all(s);
    const float r = __builtin_sqrtf(ss / float(D) + p.eps);
    const float y0 = (x0 / r) * w[lane];
    const float y1 = (x1 / r) * w[lane + 64];
    const float c0 = p.rope_cos[size_t(pos) * (D / 2) + lane];
    const float s0 = p.rope_sin[size_t(pos) * (D / 2) + lane];
    const float a = y0 * c0 - y1 * s0;
    const float b = y1 * c0 + y0 * s0;
    if (is_q) {
        float* qd = p.q + size_t(m) * p.heads * D + size_t(slot) * D;
        qd[lane] = a;
        qd[lane + 64] = b;
    } else {
        uint16_t* kdst = p.keys + size_t(pos) * p.time_stride + size_t(slot - p.heads) * D;
        kdst[lane] = f32_to_f16(a);
        kdst[lane + 64] = f32_to_f16(b);
    }
}

__global__ void prefill_position_kernel(int32_t* position, int value) { *position = value; }

// Workspace layout for a model and KV capacity.
struct PrefillLayout {
    size_t x, q8, act, qkv, qh, att, proj, gu, gemm, attn_counters, attn_part, total;
    int kp, max_chunks, qkv_rows, qd;
};

static size_t al256p(size_t v) { return (v + 255) & ~size_t(255); }

static PrefillLayout prefill_layout(const hq_model* m, int capacity)
{
    PrefillLayout L{};
    const int B = kPrefillBatch;
    const int H = m->hidden, I = m->intermediate, D = m->head_dim;
    L.qd = m->heads * D;
    L.qkv_rows = L.qd + 2 * m->kv_heads * D;
    int kmax = H > L.qd ? H : L.qd;
    if (I > kmax) kmax = I;
    L.kp = gemm_padded_k(kmax);
    L.max_chunks = (capacity + kAttnChunk - 1) / kAttnChunk;
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t at = off; off += al256p(bytes); return at; };
    L.x = take(size_t(B) * H * 4);
    L.q8 = take(size_t(gemm_padded_m(B)) * L.kp);
    L.act = take(size_t(B) * 4);
    L.qkv = take(size_t(B) * L.qkv_rows * 4);
    L.qh = take(size_t(B) * L.qd * 4);
    L.att = take(size_t(B) * L.qd * 4);
    L.proj = take(size_t(B) * H * 4);
    L.gu = take(size_t(B) * 2 * I * 4);
    size_t g = gemm_scratch_bytes(B, L.qkv_rows, H);
    g = std::max<size_t>(g, gemm_scratch_bytes(B, H, L.qd));
    g = std::max<size_t>(g, gemm_scratch_bytes(B, 2 * I, H));
    g = std::max<size_t>(g, gemm_scratch_bytes(B, H, I));
    L.gemm = take(g);
    L.attn_counters = take(size_t(B) * m->kv_heads * 4);
    L.attn_part = take(size_t(B) * attention_workspace_floats(m->heads, L.max_chunks, D) * 4);
    L.total = off;
    return L;
}

static bool prefill_fits(const hq_model* m)
{
    return m && m->layer && m->head_dim == 128 && m->kv_heads > 0 && m->heads % m->kv_heads == 0 &&
           m->heads / m->kv_heads <= 8 && (m->hidden & 31) == 0 && (m->intermediate & 31) == 0 &&
           m->intermediate <= kPrefillMaxWidth &&
           m->hidden > 0 && m->intermediate > 0 && m->vocab > 0;
}

// The GEMM reads row m of its activations at m * gemm_padded_k(width): the
// row stride follows each projection's own width.
static int run_rows(int mode, RowParams p, int rows, hipStream_t s)
{
    p.kp = gemm_padded_k(p.k);
    switch (mode) {
    case ROW_NORM: hipLaunchKernelGGL(prefill_rows_kernel<ROW_NORM>, dim3(rows), dim3(kBlock), 0, s, p); break;
    case ROW_RESID_NORM:
        hipLaunchKernelGGL(prefill_rows_kernel<ROW_RESID_NORM>, dim3(rows), dim3(kBlock), 0, s, p);
        break;
    case ROW_PLAIN: hipLaunchKernelGGL(prefill_rows_kernel<ROW_PLAIN>, dim3(rows), dim3(kBlock), 0, s, p); break;
    default: hipLaunchKernelGGL(prefill_rows_kernel<ROW_SWIGLU>, dim3(rows), dim3(kBlock), 0, s, p); break;
    }
    return hipGetLastError() == hipSuccess ? HQ_OK : HQ_ERR_LAUNCH;
}

}  // namespace hq

using namespace hq;

extern "C" size_t hq_prefill_workspace_bytes(const hq_model* model, int capacity)
{
    if (!prefill_fits(model) || capacity <= 0) return 0;
    return prefill_layout(model, capacity).total;
}

extern "C" int hq_prefill(const hq_model* m, const hq_state* st, const int32_t* tokens, int count, int start,
                          void* workspace, void* stream)
{
    if (!prefill_fits(m) || !st || !tokens || !workspace || count < 0 || start < 0) return HQ_ERR_ARG;
    if (start + count > st->capacity || start + count > m->rope_positions) return HQ_ERR_ARG;
    if (reinterpret_cast<uintptr_t>(workspace) & 255u) return HQ_ERR_ALIGN;
    if (count == 0) return HQ_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const PrefillLayout L = prefill_layout(m, st->capacity);
    char* ws = static_cast<char*>(workspace);
    float* x = reinterpret_cast<float*>(ws + L.x);
    int8_t* q8 = reinterpret_cast<int8_t*>(ws + L.q8);
    float* act = reinterpret_cast<float*>(ws + L.act);
    float* qkv = reinterpret_cast<float*>(ws + L.qkv);
    float* qh = reinterpret_cast<float*>(ws + L.qh);
    float* att = reinterpret_cast<float*>(ws + L.att);
    float* proj = reinterpret_cast<float*>(ws + L.proj);
    float* gu = reinterpret_cast<float*>(ws + L.gu);
    char* gemm = ws + L.gemm;
    const int H = m->hidden, I = m->intermediate, D = m->head_dim, KV = m->kv_heads;
    const long long time_stride = (long long)KV * D;
    const size_t layer_stride = size_t(st->capacity) * KV * D;
    const int slots = (m->heads + 2 * KV + kBlock / kWave - 1) / (kBlock / kWave);
    for (int b0 = 0; b0 < count; b0 += kPrefillBatch) {
        const int rows = count - b0 < kPrefillBatch ? count - b0 : kPrefillBatch;
        const int p0 = start + b0;
        hipLaunchKernelGGL(prefill_embed_kernel, dim3(rows), dim3(kBlock), 0, s, m->embedding, m->embedding_scales,
                           m->vocab, H, tokens + b0, st->status, x);
        if (hipGetLastError() != hipSuccess) return HQ_ERR_LAUNCH;
        for (int l = 0; l < m->layers; ++l) {
            const hq_layer& Ly = m->layer[l];
            RowParams rp{};
            rp.eps = m->eps;
            rp.q = q8;
            rp.act = act;
            // input RMSNorm (adding the previous layer's down output first)
            rp.x = x;
            rp.add = proj;
            rp.gamma = Ly.input_norm;
            rp.k = H;
            int e = run_rows(l == 0 ? ROW_NORM : ROW_RESID_NORM, rp, rows, s);
            if (e) return e;
            if (gemm_run(q8, act, Ly.qkv, Ly.qkv_scales, qkv, rows, L.qkv_rows, H, gemm, s) != hipSuccess)
                return HQ_ERR_LAUNCH;
            QkParams qp{};
            qp.qkv = qkv;
            qp.q_norm = Ly.q_norm;
            qp.k_norm = Ly.k_norm;
            qp.rope_cos = m->rope_cos;
            qp.rope_sin = m->rope_sin;
            qp.eps = m->eps;
            qp.heads = m->heads;
            qp.kv_heads = KV;
            qp.start = p0;
            qp.time_stride = time_stride;
            qp.keys = st->keys + size_t(l) * layer_stride;
            qp.values = st->values + size_t(l) * layer_stride;
            qp.q = qh;
            hipLaunchKernelGGL(prefill_qk_kernel, dim3(rows, slots), dim3(kBlock), 0, s, qp);
            if (hipGetLastError() != hipSuccess) return HQ_ERR_LAUNCH;
            AttnParams a{};
            a.q = qh;
            a.keys = qp.keys;
            a.values = qp.values;
            a.time_stride = time_stride;
            a.context = p0 + 1;
            a.batch = rows;
            a.kv_heads = KV;
            a.groups = m->heads / KV;
            a.head_dim = D;
            a.max_chunks = L.max_chunks;
            a.counters = reinterpret_cast<int32_t*>(ws + L.attn_counters);
            a.part = reinterpret_cast<float*>(ws + L.attn_part);
            a.out = att;
            if (launch_attention(a, false, s) != hipSuccess) return HQ_ERR_LAUNCH;
            // o projection, residual, post-attention RMSNorm, gate_up
            rp.x = att;
            rp.add = nullptr;
            rp.gamma = nullptr;
            rp.k = m->heads * D;
            if ((e = run_rows(ROW_PLAIN, rp, rows, s))) return e;
            if (gemm_run(q8, act, Ly.o, Ly.o_scales, proj, rows, H, rp.k, gemm, s) != hipSuccess) return HQ_ERR_LAUNCH;
            rp.x = x;
            rp.add = proj;
            rp.gamma = Ly.post_norm;
            rp.k = H;
            if ((e = run_rows(ROW_RESID_NORM, rp, rows, s))) return e;
            if (gemm_run(q8, act, Ly.gate_up, Ly.gate_up_scales, gu, rows, 2 * I, H, gemm, s) != hipSuccess)
                return HQ_ERR_LAUNCH;
            // SwiGLU, down (its residual is added at the next layer's input;
            // the last layer's is not needed: no logits for these tokens)
            rp.x = nullptr;
            rp.add = nullptr;
            rp.gate_up = gu;
            rp.gamma = nullptr;
            rp.k = I;
            if ((e = run_rows(ROW_SWIGLU, rp, rows, s))) return e;
            if (gemm_run(q8, act, Ly.down, Ly.down_scales, proj, rows, H, I, gemm, s) != hipSuccess)
                return HQ_ERR_LAUNCH;
        }
    }
    hipLaunchKernelGGL(prefill_position_kernel, dim3(1), dim3(1), 0, s, st->position, start + count);
    return hipGetLastError() == hipSuccess ? HQ_OK : HQ_ERR_LAUNCH;
}
