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
//
// The batched decode step (hq_decode_batch) runs the same layer sequence for
// the current token of up to kMaxDecodeBatch independent sequences, each
// with its own KV cache and position (a per-sequence pointer table in the
// workspace), then the final RMSNorm, the tied LM head as one GEMM over the
// batch and a per-sequence argmax that feeds each greedy token back on the
// device: M forward_token steps (cpu_lightspark.py:424-468) sharing every
// weight read, bit-identical to them.  Where the shapes allow, each layer is
// four launches (up to 8 sequences; five beyond): the qkv GEMM and the
// attention in one (separate beyond 8, where one attention block per
// sequence and kv head combines and, with the sequence's other kv-head
// blocks, quantizes the row), the attention's last blocks combining and
// quantizing each sequence's row; the o GEMM, whose last
// blocks add the residual and run the post-attention norm and
// quantization; the gate_up GEMM with SwiGLU, whose last blocks quantize
// the down input; the down GEMM, whose last blocks add the residual and run
// the next layer's input norm (the row, combine and quantization kernels
// otherwise).
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

// One token (block) per row: the prologue of the step's GEMVs.  Thread t
// holds elements t, t+THREADS, ... of the row in registers (NPT of them, all
// loaded at once, the norm weights with them), so the row is read from
// memory once.  RMSNorm (256 threads): partial t is the fmaf chain over the
// thread's elements in ascending order, and every wave folds the 256
// partials with the spec's halving tree (levels 128 and 64 from LDS, then
// the wave tree); the row is normalized, its absolute maximum taken (an
// order-free reduction, so SwiGLU rows use 1024 threads) and every
// element quantized from the registers.  The barriers wait for LDS only, and
// the updated residual row is stored last, so no barrier waits on it.
template <int MODE, int NPT, int THREADS>
__global__ __launch_bounds__(THREADS) void prefill_rows_kernel(RowParams p)
{
    constexpr bool kNorm = MODE == ROW_NORM || MODE == ROW_RESID_NORM;
    static_assert(!kNorm || THREADS == kBlock, "the RMSNorm tree takes 256 partials");
    __shared__ float red[kNorm ? kBlock : 1];
    __shared__ float wmax[THREADS / kWave];
    const int m = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int k = p.k;
    float v[NPT];
    if constexpr (MODE == ROW_SWIGLU) {
        const float* g = p.gate_up + size_t(m) * 2 * k;
        float gv[NPT], uv[NPT];
#pragma unroll
        for (int j = 0; j < NPT; ++j) {
            const int i = tid + THREADS * j;
            gv[j] = i < k ? g[i] : 0.0f;
            uv[j] = i < k ? g[k + i] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < NPT; ++j) {
            const float t = 1.0f + spec_expf(-gv[j]);
            v[j] = (gv[j] / t) * uv[j];
        }
    } else {
        float* xr = p.x + size_t(m) * k;
        float gam[kNorm ? NPT : 1];
#pragma unroll
        for (int j = 0; j < NPT; ++j) {
            const int i = tid + THREADS * j;
            v[j] = i < k ? xr[i] : 0.0f;
            if constexpr (kNorm) gam[j] = i < k ? p.gamma[i] : 0.0f;
        }
        float sum[MODE == ROW_RESID_NORM ? NPT : 1];
        if constexpr (MODE == ROW_RESID_NORM) {
            const float* ar = p.add + size_t(m) * k;
#pragma unroll
            for (int j = 0; j < NPT; ++j) {
                const int i = tid + THREADS * j;
                v[j] = i < k ? v[j] + ar[i] : 0.0f;
                sum[j] = v[j];
            }
        }
        if constexpr (kNorm) {
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < NPT; ++j)
                if (tid + THREADS * j < k) ss = __builtin_fmaf(v[j], v[j], ss);
            red[tid] = ss;
            lds_sync();
            const float r2 = (red[lane] + red[lane + 128]) + (red[lane + 64] + red[lane + 192]);
            const float total = wave_tree_sum64_all(r2);
            const float r = __builtin_sqrtf(total / float(k) + p.eps);
#pragma unroll
            for (int j = 0; j < NPT; ++j) v[j] = tid + THREADS * j < k ? (v[j] / r) * gam[j] : 0.0f;
        }
        if constexpr (MODE == ROW_RESID_NORM) {
#pragma unroll
            for (int j = 0; j < NPT; ++j) {
                const int i = tid + THREADS * j;
                if (i < k) xr[i] = sum[j];
            }
        }
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < NPT; ++j) amax = fmaxf(amax, fabsf(v[j]));   // 0 past k
    amax = wave_max64_all(amax);
    if (lane == 0) wmax[tid / kWave] = amax;
    lds_sync();
    amax = wmax[0];
#pragma unroll
    for (int w = 1; w < THREADS / kWave; ++w) amax = fmaxf(amax, wmax[w]);
    amax = fmaxf(amax, 1e-5f);
    const float inv = 127.0f / amax;
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
        const int i = tid + THREADS * j;
        if (i < k) p.q[bq_pos(m, deint_offset(i), p.kp)] = quant_i8(v[j], inv);
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
    size_t x, q8, act, qkv, qh, att, proj, gu, gemm, attn_part, total;
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

// The batched step's attention epilogue holds a row of up to 64 heads; its
// gate_up GEMM with the SwiGLU epilogue takes rows of up to 4096 columns.
static bool batch_fits(const hq_model* m) { return prefill_fits(m) && m->heads <= 64 && m->hidden <= 4096; }

// The GEMM reads row m of its activations at m * gemm_padded_k(width): the
// row stride follows each projection's own width.  Rows of up to 2560, 4096
// and 10240 values take 10, 16 and 40 registers per thread.
template <int MODE>
static void launch_rows(const RowParams& p, int rows, hipStream_t s)
{
    if constexpr (MODE != ROW_SWIGLU) {
        if (p.k <= kBlock * 10)
            hipLaunchKernelGGL((prefill_rows_kernel<MODE, 10, kBlock>), dim3(rows), dim3(kBlock), 0, s, p);
        else if (p.k <= kBlock * 16)
            hipLaunchKernelGGL((prefill_rows_kernel<MODE, 16, kBlock>), dim3(rows), dim3(kBlock), 0, s, p);
        else
            hipLaunchKernelGGL((prefill_rows_kernel<MODE, 40, kBlock>), dim3(rows), dim3(kBlock), 0, s, p);
    } else {
        // SwiGLU: 16 waves share the row's exp / divide work (its maximum
        // is order-free); 9.6 -> 6.0 us for 8 rows of 9728 against 256 threads
        constexpr int T = 4 * kBlock;
        if (p.k <= T * 4)
            hipLaunchKernelGGL((prefill_rows_kernel<MODE, 4, T>), dim3(rows), dim3(T), 0, s, p);
        else
            hipLaunchKernelGGL((prefill_rows_kernel<MODE, 10, T>), dim3(rows), dim3(T), 0, s, p);
    }
}

static int run_rows(int mode, RowParams p, int rows, hipStream_t s)
{
    if (p.k > kBlock * 40) return HQ_ERR_ARG;
    p.kp = gemm_padded_k(p.k);
    switch (mode) {
    case ROW_NORM: launch_rows<ROW_NORM>(p, rows, s); break;
    case ROW_RESID_NORM: launch_rows<ROW_RESID_NORM>(p, rows, s); break;
    case ROW_PLAIN: launch_rows<ROW_PLAIN>(p, rows, s); break;
    default: launch_rows<ROW_SWIGLU>(p, rows, s); break;
    }
    return hipGetLastError() == hipSuccess ? HQ_OK : HQ_ERR_LAUNCH;
}


// ---- batched decode step ----------------------------------------------------------

// The start of a batched step in one launch: block 0 copies the step's
// table into the workspace and advances the step counter (when the counter
// wraps past kEpochSteps - 1, or holds a value outside 0 .. kEpochSteps - 1,
// it first clears the `entry_words` 16-byte words of {value, epoch} entries
// at `entries` and restarts the count at 1); block m decodes
// sequence m's embedding row into x (a token outside the vocabulary is
// flagged and replaced by 0, a full cache flagged, as the single step's
// embedding kernel does) and runs the first layer's input RMSNorm and
// quantization on it (the
// row kernel's NORM mode: 256 strided fmaf partials, halving tree, the
// maximum over the four waves, quant_i8, de-interleaved row, act = amax/127).
template <int NPT>
__global__ __launch_bounds__(kBlock) void batch_begin_kernel(BatchTable t, BatchTable* dst, uint32_t* step_ctr,
                                                             uint4* entries, size_t entry_words, const uint8_t* emb, const float* emb_scales, int vocab,
                                                             int hidden, float* x, const float* gamma, float eps,
                                                             int8_t* q, int kq, float* act)
{
    __shared__ float red[kBlock];
    __shared__ float wmax[kBlock / kWave];
    const int m = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    if (m == 0) {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(&t);
        uint32_t* d = reinterpret_cast<uint32_t*>(dst);
        for (int i = tid; i < int(sizeof(BatchTable) / 4); i += kBlock) d[i] = src[i];
        const uint32_t c = *step_ctr + 1u;
        const bool wrap = c >= kEpochSteps || c == 0u;
        if (wrap)
            for (size_t i = tid; i < entry_words; i += kBlock) entries[i] = make_uint4(0, 0, 0, 0);
        __syncthreads();   // every thread has read the counter
        if (tid == 0) *step_ctr = wrap ? 1u : c;
    }
    int tok = *t.token[m];
    const int pos = *t.position[m];
    if (tid == 0 && (pos < 0 || pos >= t.capacity[m])) atomicOr(t.status[m], HQ_STEP_FULL);
    if (tok < 0 || tok >= vocab) {
        if (tid == 0) atomicOr(t.status[m], HQ_STEP_BAD_TOKEN);
        tok = 0;
    }
    const uint8_t* row = emb + size_t(tok) * size_t(hidden >> 1);
    const float sc = emb_scales[tok];
    float* xr = x + size_t(m) * hidden;
    float v[NPT], gam[NPT];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
        const int i = tid + kBlock * j;
        if (i < hidden) {
            const uint8_t byte = row[i >> 1];
            const int nib = (i & 1) ? int(int8_t(byte)) >> 4 : int(int8_t(uint8_t(byte << 4))) >> 4;
            v[j] = float(nib) * sc;
            gam[j] = gamma[i];
            xr[i] = v[j];
            ss = __builtin_fmaf(v[j], v[j], ss);
        } else {
            v[j] = 0.0f;
            gam[j] = 0.0f;
        }
    }
    red[tid] = ss;
    lds_sync();
    const float r2 = (red[lane] + red[lane + 128]) + (red[lane + 64] + red[lane + 192]);
    const float total = wave_tree_sum64_all(r2);
    const float r = __builtin_sqrtf(total / float(hidden) + eps);
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
        v[j] = tid + kBlock * j < hidden ? (v[j] / r) * gam[j] : 0.0f;
        amax = fmaxf(amax, fabsf(v[j]));
    }
    amax = wave_max64_all(amax);
    if (lane == 0) wmax[tid / kWave] = amax;
    lds_sync();
    amax = wmax[0];
#pragma unroll
    for (int w = 1; w < kBlock / kWave; ++w) amax = fmaxf(amax, wmax[w]);
    amax = fmaxf(amax, 1e-5f);
    const float inv = 127.0f / amax;
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
        const int i = tid + kBlock * j;
        if (i < hidden) q[bq_pos(m, deint_offset(i), kq)] = quant_i8(v[j], inv);
    }
    if (tid == 0) act[m] = amax / 127.0f;
}

// Block (b, m): logits [b*kArgPer, ...) of sequence m copied to its state's
// logits and reduced to a (value, index) partial with np.argmax's order; the
// last block of the row (two-level ticket) writes the greedy token and
// advances the position, as the single step's LM head does.
constexpr int kBatchArgPer = kBlock * 16;
__global__ __launch_bounds__(kBlock) void batch_argmax_kernel(const float* logits, int vocab, const BatchTable* T,
                                                              float* pval, int32_t* pidx, int32_t* counters)
{
    __shared__ float sv[kBlock / kWave];
    __shared__ int si[kBlock / kWave];
    __shared__ int last_flag;
    const int tid = threadIdx.x;
    const int m = blockIdx.y;
    const int nb = gridDim.x;
    const float* row = logits + size_t(m) * size_t(vocab);
    float* dst = T->logits[m];
    float v = -__builtin_inff();
    int idx = 0x7FFFFFFF;
    const int base = blockIdx.x * kBatchArgPer;
    for (int i = base + tid; i < min(vocab, base + kBatchArgPer); i += kBlock) {
        const float x = row[i];
        dst[i] = x;
        if (argmax_better(x, i, v, idx)) { v = x; idx = i; }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(v, o, kWave);
        const int oi = __shfl_xor(idx, o, kWave);
        if (argmax_better(ov, oi, v, idx)) { v = ov; idx = oi; }
    }
    if ((tid & (kWave - 1)) == 0) { sv[tid / kWave] = v; si[tid / kWave] = idx; }
    __syncthreads();
    float* pv = pval + size_t(m) * nb;
    int32_t* pi = pidx + size_t(m) * nb;
    if (tid == 0) {
        for (int w = 1; w < kBlock / kWave; ++w)
            if (argmax_better(sv[w], si[w], v, idx)) { v = sv[w]; idx = si[w]; }
        publish_f(pv + blockIdx.x, v);
        publish_i(pi + blockIdx.x, idx);
        wait_all_memory();
        last_flag = last_block_ticket(counters + size_t(m) * ticket_words(nb), blockIdx.x, nb);
    }
    __syncthreads();
    if (!last_flag) return;
    v = -__builtin_inff();
    idx = 0x7FFFFFFF;
    for (int b = tid; b < nb; b += kBlock) {
        const float bv = read_f(pv + b);
        const int bi = read_i(pi + b);
        if (argmax_better(bv, bi, v, idx)) { v = bv; idx = bi; }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(v, o, kWave);
        const int oi = __shfl_xor(idx, o, kWave);
        if (argmax_better(ov, oi, v, idx)) { v = ov; idx = oi; }
    }
    __syncthreads();
    if ((tid & (kWave - 1)) == 0) { sv[tid / kWave] = v; si[tid / kWave] = idx; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kBlock / kWave; ++w)
            if (argmax_better(sv[w], si[w], v, idx)) { v = sv[w]; idx = si[w]; }
        *T->token[m] = idx;
        const int pos = *T->position[m];
        if (pos >= 0 && pos < T->capacity[m]) *T->position[m] = pos + 1;
    }
}

// The batch's residual rows back into each state's x (the single step leaves
// the final residual there).
__global__ __launch_bounds__(kBlock) void batch_store_x_kernel(const float* x, int hidden, const BatchTable* T)
{
    const int m = blockIdx.x;
    for (int i = threadIdx.x; i < hidden; i += kBlock) T->x[m][i] = x[size_t(m) * hidden + i];
}

struct BatchLayout {
    size_t x, q8, act, qkv, att, proj, gu, gemm, attn_part, logits, pval, pidx, tickets, pmax, table, ll,
        pmax_ll, ll_part, ll_out, ll_max, step_ctr, total;
    int kp, max_chunks, qkv_rows, qd, arg_blocks;
};

static BatchLayout batch_layout(const hq_model* m, int max_capacity)
{
    BatchLayout L{};
    const int B = kMaxDecodeBatch;
    const int H = m->hidden, I = m->intermediate, D = m->head_dim, V = m->vocab;
    L.qd = m->heads * D;
    L.qkv_rows = L.qd + 2 * m->kv_heads * D;
    int kmax = H > L.qd ? H : L.qd;
    if (I > kmax) kmax = I;
    L.kp = gemm_padded_k(kmax);
    L.max_chunks = (max_capacity + kAttnChunk - 1) / kAttnChunk;
    L.arg_blocks = (V + kBatchArgPer - 1) / kBatchArgPer;
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t at = off; off += al256p(bytes); return at; };
    L.step_ctr = take(4);   // first: the step counter sits at offset 0 (include/hq.h)
    L.x = take(size_t(B) * H * 4);
    L.q8 = take(size_t(gemm_padded_m(B)) * L.kp);
    L.act = take(size_t(B) * 4);
    L.qkv = take(size_t(B) * L.qkv_rows * 4);
    L.att = take(size_t(B) * L.qd * 4);
    L.proj = take(size_t(B) * H * 4);
    L.gu = take(size_t(B) * 2 * I * 4);
    size_t g = gemm_scratch_bytes(B, L.qkv_rows, H);
    g = std::max<size_t>(g, gemm_scratch_bytes(B, H, L.qd));
    g = std::max<size_t>(g, gemm_scratch_bytes(B, 2 * I, H));
    g = std::max<size_t>(g, gemm_scratch_bytes(B, H, I));
    g = std::max<size_t>(g, gemm_scratch_bytes(B, V, H));
    L.gemm = take(g);
    L.attn_part = take(size_t(B) * attention_workspace_floats(m->heads, L.max_chunks, D) * 4);
    L.logits = take(size_t(B) * V * 4);
    L.pval = take(size_t(B) * L.arg_blocks * 4);
    L.pidx = take(size_t(B) * L.arg_blocks * 4);
    L.tickets = take(size_t(B) * ticket_words(L.arg_blocks) * 4);
    L.pmax = take(size_t(gemm_swiglu_blocks(I)) * B * 4);
    L.table = take(sizeof(BatchTable));
    // the {value, epoch} entries, contiguous to the end (cleared together
    // when the step counter wraps)
    L.ll = take(size_t(B) * std::max(std::max(H, I), L.qkv_rows) * 8);
    L.ll_part = take(size_t(B) * attention_workspace_floats(m->heads, L.max_chunks, D) * 8);
    L.ll_out = take(size_t(B) * L.qd * 8);
    L.ll_max = take(size_t(B) * 8 * 8);
    L.pmax_ll = take(size_t(gemm_swiglu_blocks(I)) * B * 8);
    L.total = off;
    return L;
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

extern "C" size_t hq_decode_batch_workspace_bytes(const hq_model* model, int max_capacity)
{
    if (!batch_fits(model) || max_capacity <= 0) return 0;
    return batch_layout(model, max_capacity).total;
}

extern "C" int hq_decode_batch(const hq_model* m, const hq_state* states, int count, int max_capacity,
                               void* workspace, void* stream)
{
    if (!batch_fits(m) || !states || !workspace || count < 1 || count > kMaxDecodeBatch || max_capacity <= 0)
        return HQ_ERR_ARG;
    if (reinterpret_cast<uintptr_t>(workspace) & 255u) return HQ_ERR_ALIGN;
    if (!m->embedding || !m->embedding_scales || !m->final_norm || !m->rope_cos || !m->rope_sin) return HQ_ERR_ARG;
    BatchTable t{};
    t.count = count;
    for (int i = 0; i < count; ++i) {
        const hq_state& st = states[i];
        if (st.capacity <= 0 || st.capacity > max_capacity || st.capacity > m->rope_positions) return HQ_ERR_ARG;
        if (!st.keys || !st.values || !st.position || !st.token || !st.status || !st.x || !st.logits)
            return HQ_ERR_ARG;
        if ((reinterpret_cast<uintptr_t>(st.keys) & 15u) || (reinterpret_cast<uintptr_t>(st.values) & 15u))
            return HQ_ERR_ALIGN;
        t.keys[i] = st.keys;
        t.values[i] = st.values;
        t.position[i] = st.position;
        t.token[i] = st.token;
        t.status[i] = st.status;
        t.x[i] = st.x;
        t.logits[i] = st.logits;
        t.capacity[i] = st.capacity;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    const BatchLayout L = batch_layout(m, max_capacity);
    char* ws = static_cast<char*>(workspace);
    float* x = reinterpret_cast<float*>(ws + L.x);
    int8_t* q8 = reinterpret_cast<int8_t*>(ws + L.q8);
    float* act = reinterpret_cast<float*>(ws + L.act);
    float* qkv = reinterpret_cast<float*>(ws + L.qkv);
    float* att = reinterpret_cast<float*>(ws + L.att);
    float* proj = reinterpret_cast<float*>(ws + L.proj);
    float* gu = reinterpret_cast<float*>(ws + L.gu);
    float* logits = reinterpret_cast<float*>(ws + L.logits);
    char* gemm = ws + L.gemm;
    BatchTable* table = reinterpret_cast<BatchTable*>(ws + L.table);
    const int H = m->hidden, I = m->intermediate, D = m->head_dim, KV = m->kv_heads, M = count;
    const long long time_stride = (long long)KV * D;
    auto ok = [] { return hipGetLastError() == hipSuccess; };
    uint32_t* step_ctr = reinterpret_cast<uint32_t*>(ws + L.step_ctr);
    uint4* entries = reinterpret_cast<uint4*>(ws + L.ll);
    const size_t entry_words = (L.total - L.ll) / 16;
    // the table, the embedding rows and the first layer's input rows
    if (H <= kBlock * 10)
        hipLaunchKernelGGL((batch_begin_kernel<10>), dim3(M), dim3(kBlock), 0, s, t, table, step_ctr, entries,
                           entry_words, m->embedding, m->embedding_scales, m->vocab, H, x, m->layer[0].input_norm,
                           m->eps, q8, gemm_padded_k(H), act);
    else
        hipLaunchKernelGGL((batch_begin_kernel<16>), dim3(M), dim3(kBlock), 0, s, t, table, step_ctr, entries,
                           entry_words, m->embedding, m->embedding_scales, m->vocab, H, x, m->layer[0].input_norm,
                           m->eps, q8, gemm_padded_k(H), act);
    if (!ok()) return HQ_ERR_LAUNCH;
    RowParams rp{};
    rp.eps = m->eps;
    rp.q = q8;
    rp.act = act;
    int e;
    // The o and down GEMMs finish the next GEMM's input rows in their tails
    // (residual add, RMSNorm, quantization) where the shapes allow, instead
    // of a row kernel after them.
    const bool tails = m->layers <= 64 && gemm_tail_fits(M, H, L.qd) && gemm_tail_fits(M, H, I);
    const bool swiglu_tail = tails && gemm_swiglu_tail_fits(M, I, H);
    GemmTail tl{};
    tl.pmax = reinterpret_cast<uint64_t*>(ws + L.pmax_ll);
    tl.ll = reinterpret_cast<uint64_t*>(ws + L.ll);
    tl.epoch_ctr = step_ctr;
    tl.x = x;
    tl.eps = m->eps;
    tl.q = q8;
    tl.act = act;
    tl.table = table;
    for (int l = 0; l < m->layers; ++l) {
        const hq_layer& Ly = m->layer[l];
        rp.x = x;
        rp.add = proj;
        rp.gate_up = nullptr;
        rp.gamma = Ly.input_norm;
        rp.k = H;
        if (l > 0 && !tails && (e = run_rows(ROW_RESID_NORM, rp, M, s))) return e;
        // the qkv GEMM; q/k head norms, RoPE and the K/V write of each
        // sequence inside the attention kernel; its output rows combined and
        // quantized for o (the GEMM and the attention in one launch where the
        // tails apply)
        AttnParams a{};
        a.qkv = qkv;
        a.q_norm = Ly.q_norm;
        a.k_norm = Ly.k_norm;
        a.rope_cos = m->rope_cos;
        a.rope_sin = m->rope_sin;
        a.eps = m->eps;
        a.time_stride = time_stride;
        a.batch = M;
        a.kv_heads = KV;
        a.groups = m->heads / KV;
        a.head_dim = D;
        a.max_chunks = L.max_chunks;
        a.part = reinterpret_cast<float*>(ws + L.attn_part);
        a.out = att;
        a.table = table;
        a.layer = l;
        a.q8 = q8;
        a.act = act;
        a.kp = gemm_padded_k(L.qd);
        if (tails) {
            a.ll_part = reinterpret_cast<uint64_t*>(ws + L.ll_part);
            a.ll_out = reinterpret_cast<uint64_t*>(ws + L.ll_out);
            a.ll_max = reinterpret_cast<uint64_t*>(ws + L.ll_max);
            a.epoch_ctr = step_ctr;
            a.epoch_id = 4 * l;   // (unique per launch of the step: the launches share L.ll)
            a.qkv_ll = reinterpret_cast<uint64_t*>(ws + L.ll);
        }
        hipError_t fe = hipErrorNotSupported;
        if (tails) fe = launch_batch_qkv_attention(q8, act, Ly.qkv, Ly.qkv_scales, H, a, s);
        if (fe == hipErrorNotSupported) {
            a.qkv_ll = nullptr;
            if (gemm_run(q8, act, Ly.qkv, Ly.qkv_scales, qkv, M, L.qkv_rows, H, gemm, s) != hipSuccess)
                return HQ_ERR_LAUNCH;
            if (launch_batch_attention(a, s) != hipSuccess) return HQ_ERR_LAUNCH;
        } else if (fe != hipSuccess) {
            return HQ_ERR_LAUNCH;
        }
        if (tails) {
            tl.epoch_id = 4 * l + 1;
            tl.gamma = Ly.post_norm;
            tl.kq = gemm_padded_k(H);
            if (gemm_run_tail(q8, act, Ly.o, Ly.o_scales, M, H, L.qd, tl, s) != hipSuccess) return HQ_ERR_LAUNCH;
        } else {
            if (gemm_run(q8, act, Ly.o, Ly.o_scales, proj, M, H, L.qd, gemm, s) != hipSuccess) return HQ_ERR_LAUNCH;
            rp.x = x;
            rp.add = proj;
            rp.gamma = Ly.post_norm;
            rp.k = H;
            if ((e = run_rows(ROW_RESID_NORM, rp, M, s))) return e;
        }
        // gate_up with SwiGLU in its epilogue, then the down input's quant
        // (in its tail where it has one)
        if (swiglu_tail) {
            tl.epoch_id = 4 * l + 2;
            tl.kq = gemm_padded_k(I);
            if (gemm_run_swiglu_tail(q8, act, Ly.gate_up, Ly.gate_up_scales, M, I, H, tl, s) != hipSuccess)
                return HQ_ERR_LAUNCH;
        } else if (gemm_run_swiglu(q8, act, Ly.gate_up, Ly.gate_up_scales, gu, M, I, H,
                                   reinterpret_cast<float*>(ws + L.pmax), q8, gemm_padded_k(I), act, s) != hipSuccess) {
            return HQ_ERR_LAUNCH;
        }
        if (tails) {
            // the next layer's input rows (the final norm's after the last layer)
            tl.epoch_id = 4 * l + 3;
            tl.gamma = l + 1 < m->layers ? m->layer[l + 1].input_norm : m->final_norm;
            tl.kq = gemm_padded_k(H);
            if (gemm_run_tail(q8, act, Ly.down, Ly.down_scales, M, H, I, tl, s) != hipSuccess) return HQ_ERR_LAUNCH;
        } else if (gemm_run(q8, act, Ly.down, Ly.down_scales, proj, M, H, I, gemm, s) != hipSuccess) {
            return HQ_ERR_LAUNCH;
        }
    }
    // the last layer's down output into the residual, final RMSNorm (in the
    // last down GEMM's tail where it has one), tied LM head over the batch,
    // per-sequence argmax and position advance
    rp.x = x;
    rp.add = proj;
    rp.gate_up = nullptr;
    rp.gamma = m->final_norm;
    rp.k = H;
    if (!tails && (e = run_rows(ROW_RESID_NORM, rp, M, s))) return e;
    if (gemm_run(q8, act, m->embedding, m->embedding_scales, logits, M, m->vocab, H, gemm, s) != hipSuccess)
        return HQ_ERR_LAUNCH;
    hipLaunchKernelGGL(batch_argmax_kernel, dim3(L.arg_blocks, M), dim3(kBlock), 0, s, logits, m->vocab,
                       (const BatchTable*)table, reinterpret_cast<float*>(ws + L.pval),
                       reinterpret_cast<int32_t*>(ws + L.pidx), reinterpret_cast<int32_t*>(ws + L.tickets));
    hipLaunchKernelGGL(batch_store_x_kernel, dim3(M), dim3(kBlock), 0, s, x, H, (const BatchTable*)table);
    return ok() ? HQ_OK : HQ_ERR_LAUNCH;
}
