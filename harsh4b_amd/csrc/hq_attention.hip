// hq_attention.hip - fused single-token GQA decode attention for gfx950.
//
// Same mathematics as litespark_gqa_decode (cpu_kernels/litespark_int4.cpp:
// 160-259 in the reference repository): per query head, scores
// (q . k_t) / sqrt(D), softmax over t, and sum_t p_t v_t -- computed in one
// kernel over an fp16 KV cache.
//
// At batch 1 there are only kv_heads (8) independent heads, so the time axis
// is split into chunks of 64 positions: block (kv_head, chunk) handles the
// `groups` query heads that share one K/V stream (each K/V byte is read
// once), computes its chunk's max, exp-sum and partial V accumulation, and
// the last block of a kv head to arrive (an atomic ticket, no waiting)
// combines the chunk partials.  In STEP mode the kernel also applies the
// per-head RMSNorm (cpu_lightspark.py:435-436) and RoPE (:437-438) to the raw
// q/k projection and writes the fp16 k/v of the current position into the
// cache (:439-440), so no separate kernel runs between the qkv GEMV and the
// o GEMV.
//
// Spec order (bit-identical to the oracle's or_gqa_decode_split):
//   score   16 partial fmaf chains of D/16 consecutive dims, halving tree
//           over the 16 lanes, times 1/sqrt(D);
//   chunk   m = max, e_t = exp(s_t - m), l = halving tree over 64 slots,
//           o[d] = fmaf chain of e_t * v_t[d] over ascending t;
//   combine M = max m_c; a_c = exp(m_c - M); L and O[d] as fmaf chains over
//           ascending c; out = O * (1 / L).
#include "hq_device.h"
#include "hq_internal.h"

namespace hq {

template <int D>
__device__ __forceinline__ void load_k_lane(const uint16_t* src, float* k)
{
    constexpr int DPL = D / 16;
    if constexpr (DPL == 8) {
        const uint4 v = *reinterpret_cast<const uint4*>(src);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            k[2 * j] = f16_to_f32(uint16_t(w[j] & 0xFFFFu));
            k[2 * j + 1] = f16_to_f32(uint16_t(w[j] >> 16));
        }
    } else if constexpr (DPL == 4) {
        const uint2 v = *reinterpret_cast<const uint2*>(src);
        k[0] = f16_to_f32(uint16_t(v.x & 0xFFFFu));
        k[1] = f16_to_f32(uint16_t(v.x >> 16));
        k[2] = f16_to_f32(uint16_t(v.y & 0xFFFFu));
        k[3] = f16_to_f32(uint16_t(v.y >> 16));
    } else {
#pragma unroll
        for (int j = 0; j < DPL; ++j) k[j] = f16_to_f32(src[j]);
    }
}

template <int D, int GMAX, bool STEP>
__global__ __launch_bounds__(kBlock) void attention_kernel(AttnParams a)
{
    constexpr int C = kAttnChunk;
    constexpr int DPL = D / 16;
    constexpr int PAIRS = (GMAX * D + kBlock - 1) / kBlock;   // (head, dim) pairs per thread
    constexpr int HSTEP = kBlock / D;                          // heads between a thread's pairs
    __shared__ float q_s[GMAX][D];
    __shared__ float kcur[D];
    __shared__ float vcur[D];
    __shared__ float e_s[GMAX][C];
    __shared__ int last_flag;

    const int g = blockIdx.x;
    const int c = blockIdx.y;
    const int G = a.groups;
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid & (kWave - 1);

    int n, pos;
    if constexpr (STEP) {
        pos = *a.position;
        if (pos < 0 || pos >= a.capacity) {
            if (g == 0 && c == 0 && tid == 0) atomicOr(a.status, HQ_STEP_FULL);
            return;
        }
        n = pos + 1;
    } else {
        pos = -1;
        n = a.context;
    }
    const int nc = (n + C - 1) / C;
    if (c >= nc) return;
    const int t0 = c * C;
    const int tn = min(C, n - t0);          // valid positions in this chunk
    const bool has_cur = STEP && (c == nc - 1);
    const size_t kv_off = size_t(g) * D;

    // ---- phase 1: query heads (and in STEP mode the current k/v) ----------
    if constexpr (STEP) {
        static_assert(D == 128, "STEP mode is written for head_dim 128");
        const float* cs = a.rope_cos + size_t(pos) * (D / 2);
        const float* sn = a.rope_sin + size_t(pos) * (D / 2);
        for (int h = wave; h < G; h += kBlock / kWave) {
            const float* src = a.qkv + size_t(g * G + h) * D;
            const float x0 = src[lane], x1 = src[lane + 64];
            float p = __builtin_fmaf(x0, x0, 0.0f);
            p = __builtin_fmaf(x1, x1, p);
            const float ss = tree_sum<kWave>(p);
            const float r = __builtin_sqrtf(ss / float(D) + a.eps);
            const float y0 = (x0 / r) * a.q_norm[lane];
            const float y1 = (x1 / r) * a.q_norm[lane + 64];
            const float c0 = cs[lane], s0 = sn[lane];
            q_s[h][lane] = y0 * c0 - y1 * s0;
            q_s[h][lane + 64] = y1 * c0 + y0 * s0;
        }
        if (has_cur) {
            const int heads = a.kv_heads * G;
            uint16_t* kdst = a.keys + size_t(pos) * a.time_stride + kv_off;
            uint16_t* vdst = a.values + size_t(pos) * a.time_stride + kv_off;
            if (wave == 0) {
                const float* src = a.qkv + size_t(heads + g) * D;
                const float x0 = src[lane], x1 = src[lane + 64];
                float p = __builtin_fmaf(x0, x0, 0.0f);
                p = __builtin_fmaf(x1, x1, p);
                const float ss = tree_sum<kWave>(p);
                const float r = __builtin_sqrtf(ss / float(D) + a.eps);
                const float y0 = (x0 / r) * a.k_norm[lane];
                const float y1 = (x1 / r) * a.k_norm[lane + 64];
                const float c0 = cs[lane], s0 = sn[lane];
                const uint16_t h0 = f32_to_f16(y0 * c0 - y1 * s0);
                const uint16_t h1 = f32_to_f16(y1 * c0 + y0 * s0);
                kdst[lane] = h0;
                kdst[lane + 64] = h1;
                kcur[lane] = f16_to_f32(h0);
                kcur[lane + 64] = f16_to_f32(h1);
            } else if (wave == 1) {
                const float* src = a.qkv + size_t(heads + a.kv_heads + g) * D;
                const uint16_t h0 = f32_to_f16(src[lane]);
                const uint16_t h1 = f32_to_f16(src[lane + 64]);
                vdst[lane] = h0;
                vdst[lane + 64] = h1;
                vcur[lane] = f16_to_f32(h0);
                vcur[lane + 64] = f16_to_f32(h1);
            }
        }
    } else {
        for (int i = tid; i < G * D; i += kBlock) q_s[i / D][i % D] = a.q[size_t(g * G) * D + i];
    }
    __syncthreads();

    // ---- phase 2: scores, 16 lanes per position ----------------------------
    {
        const int grp = tid >> 4;       // 16 groups
        const int l16 = tid & 15;
        const float scale = 1.0f / __builtin_sqrtf(float(D));
        float qr[GMAX][DPL];
#pragma unroll
        for (int h = 0; h < GMAX; ++h)
#pragma unroll
            for (int j = 0; j < DPL; ++j) qr[h][j] = (h < G) ? q_s[h][l16 * DPL + j] : 0.0f;
#pragma unroll
        for (int rep = 0; rep < C / 16; ++rep) {
            const int i = grp + 16 * rep;
            const int t = t0 + i;
            if (i < tn) {
                float k[DPL];
                if (has_cur && t == pos) {
#pragma unroll
                    for (int j = 0; j < DPL; ++j) k[j] = kcur[l16 * DPL + j];
                } else {
                    load_k_lane<D>(a.keys + size_t(t) * a.time_stride + kv_off + l16 * DPL, k);
                }
#pragma unroll
                for (int h = 0; h < GMAX; ++h) {
                    if (h < G) {
                        float pp = 0.0f;
#pragma unroll
                        for (int j = 0; j < DPL; ++j) pp = __builtin_fmaf(qr[h][j], k[j], pp);
                        const float dot = tree_sum<16>(pp);
                        if (l16 == 0) e_s[h][i] = dot * scale;
                    }
                }
            } else if (l16 == 0) {
#pragma unroll
                for (int h = 0; h < GMAX; ++h)
                    if (h < G) e_s[h][i] = -__builtin_inff();
            }
        }
    }
    __syncthreads();

    // ---- phase 3: chunk softmax statistics, one wave per head --------------
    const int heads = a.kv_heads * G;
    const int pstride = D + 2;
    for (int h = wave; h < G; h += kBlock / kWave) {
        const float s = e_s[h][lane];
        const float m = fmax_group<kWave>(s);
        const float e = (lane < tn) ? spec_expf(s - m) : 0.0f;
        const float l = tree_sum<kWave>(e);
        e_s[h][lane] = e;
        if (lane == 0) {
            float* pp = a.part + (size_t(g * G + h) * a.max_chunks + c) * pstride;
            pp[0] = m;
            pp[1] = l;
        }
    }
    __syncthreads();

    // ---- phase 4: partial V accumulation ------------------------------------
    const int d = tid % D;
    const int h0 = tid / D;
    {
        float o[PAIRS];
#pragma unroll
        for (int r = 0; r < PAIRS; ++r) o[r] = 0.0f;
        const uint16_t* vsrc = a.values + size_t(t0) * a.time_stride + kv_off + d;
        for (int i = 0; i < tn; ++i) {
            float v;
            if (has_cur && t0 + i == pos) v = vcur[d];
            else v = f16_to_f32(vsrc[size_t(i) * a.time_stride]);
#pragma unroll
            for (int r = 0; r < PAIRS; ++r) {
                const int h = h0 + HSTEP * r;
                if (h < G) o[r] = __builtin_fmaf(e_s[h][i], v, o[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < PAIRS; ++r) {
            const int h = h0 + HSTEP * r;
            if (h < G) a.part[(size_t(g * G + h) * a.max_chunks + c) * pstride + 2 + d] = o[r];
        }
    }

    // ---- phase 5: last block of this kv head combines ----------------------
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const int ticket = atomicAdd(a.counters + g, 1);
        last_flag = (ticket == nc - 1);
    }
    __syncthreads();
    if (!last_flag) return;
    __threadfence();
#pragma unroll
    for (int r = 0; r < PAIRS; ++r) {
        const int h = h0 + HSTEP * r;
        if (h >= G) continue;
        const float* base = a.part + size_t(g * G + h) * a.max_chunks * pstride;
        float M = -__builtin_inff();
        for (int cc = 0; cc < nc; ++cc)
            M = fmaxf(M, __hip_atomic_load(base + size_t(cc) * pstride, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT));
        float L = 0.0f, O = 0.0f;
        for (int cc = 0; cc < nc; ++cc) {
            const float* pc = base + size_t(cc) * pstride;
            const float mc = __hip_atomic_load(pc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const float lc = __hip_atomic_load(pc + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const float oc = __hip_atomic_load(pc + 2 + d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const float al = spec_expf(mc - M);
            L = __builtin_fmaf(al, lc, L);
            O = __builtin_fmaf(al, oc, O);
        }
        a.out[size_t(g * G + h) * D + d] = O * (1.0f / L);
    }
    if (tid == 0) a.counters[g] = 0;
    (void)heads;
}

size_t attention_workspace_floats(int heads, int max_chunks, int head_dim)
{
    return size_t(heads) * size_t(max_chunks) * size_t(head_dim + 2);
}

template <int D, int GMAX, bool STEP>
static hipError_t launch_attn(const AttnParams& a, hipStream_t s)
{
    hipLaunchKernelGGL((attention_kernel<D, GMAX, STEP>), dim3(a.kv_heads, a.max_chunks),
                       dim3(kBlock), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_attention(const AttnParams& a, bool step_mode, hipStream_t s)
{
    if (step_mode) {
        if (a.head_dim != 128 || a.groups > 4) return hipErrorInvalidValue;
        return launch_attn<128, 4, true>(a, s);
    }
    switch (a.head_dim) {
    case 16: return launch_attn<16, 8, false>(a, s);
    case 32: return launch_attn<32, 8, false>(a, s);
    case 64: return launch_attn<64, 8, false>(a, s);
    case 128: return launch_attn<128, 8, false>(a, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace hq

using namespace hq;

extern "C" size_t hq_gqa_workspace_bytes(int context, int kv_heads, int groups, int head_dim)
{
    if (context <= 0 || kv_heads <= 0 || groups <= 0 || head_dim <= 0) return 0;
    const int nc = (context + kAttnChunk - 1) / kAttnChunk;
    // arrival counters in the first 256 bytes (a fixed place, so one zeroed
    // workspace serves every context up to the one it was sized for), then
    // the chunk partials
    return 256 + attention_workspace_floats(kv_heads * groups, nc, head_dim) * 4;
}

extern "C" int hq_gqa_decode(const float* query, const uint16_t* keys, const uint16_t* values,
                             void* workspace, float* output, int context, int kv_heads,
                             int groups, int head_dim, int kv_time_stride, void* stream)
{
    if (!query || !keys || !values || !workspace || !output) return HQ_ERR_ARG;
    if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return HQ_ERR_ALIGN;
    if (context <= 0 || kv_heads <= 0 || groups <= 0 || groups > 8) return HQ_ERR_ARG;
    if (head_dim != 16 && head_dim != 32 && head_dim != 64 && head_dim != 128) return HQ_ERR_ARG;
    if (kv_time_stride < kv_heads * head_dim) return HQ_ERR_ARG;
    if (kv_heads * 256 > 256 * 64) return HQ_ERR_ARG;   // counters fit in 256 bytes
    const size_t dpl_bytes = size_t(head_dim / 16) * 2;
    if (((reinterpret_cast<uintptr_t>(keys)) % dpl_bytes) != 0 ||
        (size_t(kv_time_stride) * 2) % dpl_bytes != 0)
        return HQ_ERR_ALIGN;
    const int nc = (context + kAttnChunk - 1) / kAttnChunk;
    AttnParams a{};
    a.q = query;
    a.keys = const_cast<uint16_t*>(keys);
    a.values = const_cast<uint16_t*>(values);
    a.time_stride = kv_time_stride;
    a.context = context;
    a.kv_heads = kv_heads;
    a.groups = groups;
    a.head_dim = head_dim;
    a.max_chunks = nc;
    a.counters = static_cast<int32_t*>(workspace);
    a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + 256);
    a.out = output;
    const hipError_t e = launch_attention(a, false, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? HQ_OK : HQ_ERR_LAUNCH;
}
