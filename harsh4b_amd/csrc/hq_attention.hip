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
// once), computes its chunk's max, exp-sum and partial V accumulation and
// publishes them; a second kernel (attention_combine_kernel) combines the
// chunk partials of every (query head, dim) in parallel.  In STEP mode the kernel also applies the
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
#include <mutex>

#include "hq_gemm_block.h"

namespace hq {

// K and V of one chunk are staged in LDS: every 16-byte load of a chunk is
// issued one chunk ahead (two register buffers), so each chunk costs one
// memory round trip at most.  Rows are padded by 16 bytes to spread banks.
template <int D>
struct ChunkTile {
    static constexpr int kRowHalves = D + 8;                 // padded row
    static constexpr int kGroupsPerRow = D / 8;              // 16-byte groups per row
    static constexpr int kGroups = kAttnChunk * kGroupsPerRow;
    static constexpr int kPerThread = (kGroups + kBlock - 1) / kBlock;
};

// (thread `tid` of a 256-thread group: the block's thread by default)
template <int D>
__device__ __forceinline__ void load_chunk(const AttnParams& a, const uint16_t* keys, const uint16_t* values,
                                           int t0, int tn, int skip_t, size_t kv_off, uint4* kreg, uint4* vreg,
                                           int tid = -1)
{
    using T = ChunkTile<D>;
    if (tid < 0) tid = int(threadIdx.x);
#pragma unroll
    for (int r = 0; r < T::kPerThread; ++r) {
        const int id = tid + kBlock * r;
        const int t = id / T::kGroupsPerRow;
        const int d8 = id % T::kGroupsPerRow;
        const bool ok = id < T::kGroups && t < tn && t != skip_t;
        const size_t off = size_t(t0 + t) * a.time_stride + kv_off + size_t(d8) * 8;
        kreg[r] = ok ? *reinterpret_cast<const uint4*>(keys + off) : make_uint4(0, 0, 0, 0);
        vreg[r] = ok ? *reinterpret_cast<const uint4*>(values + off) : make_uint4(0, 0, 0, 0);
    }
}

// Block (kv_head, split) walks chunks [split*CPB, split*CPB + CPB) of the
// context.  With a single split (context <= CPB*64) it combines its chunk
// partials itself; otherwise the partials go to the workspace and
// attention_combine_kernel combines them.  Either way the combine runs over
// ascending chunks, so the result is the same bits.

// The LDS of one attention block.
template <int D, int GMAX, int CPB>
struct AttnLds {
    float q_s[GMAX][D];
    alignas(16) uint16_t k_s[kAttnChunk * ChunkTile<D>::kRowHalves];
    alignas(16) uint16_t v_s[kAttnChunk * ChunkTile<D>::kRowHalves];
    uint16_t kc_s[D];
    uint16_t vc_s[D];
    float e_s[GMAX][kAttnChunk];
    float m_s[GMAX][CPB];
    float l_s[GMAX][CPB];
    float o_s[CPB][GMAX][D];   // per-chunk V partials
};

// Block (bx, by, bz) = (kv head, split, query) of an attention launch.
// Two raw-projection values (dims lane and lane + 64 at p) from {value,
// epoch} entries, once both are current (bounded wait).
__device__ __forceinline__ void poll_pair(const uint64_t* p, uint32_t ep, int32_t* status, float& x0, float& x1)
{
    uint64_t e0 = tail_load(p), e1 = tail_load(p + 64);
    unsigned spins = 0;
    while (!(tail_ready(e0, ep) && tail_ready(e1, ep))) {
        if (++spins == kTailSpinLimit) {
            atomicOr(status, HQ_STEP_SYNC);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
        if (!tail_ready(e0, ep)) e0 = tail_load(p);
        if (!tail_ready(e1, ep)) e1 = tail_load(p + 64);
    }
    x0 = bits_f32(uint32_t(e0));
    x1 = bits_f32(uint32_t(e1));
}

// QLL: the raw projection comes as {value, epoch} entries from the qkv GEMM
// blocks of the same launch (a.qkv_ll) instead of the qkv buffer.
template <int D, int GMAX, bool STEP, int CPB, bool TAILS, bool QLL = false>
__device__ __forceinline__ int attention_block(const AttnParams& a, uint32_t ep, AttnLds<D, GMAX, CPB>& lds,
                                               int bx, int by, int bz)
{
    constexpr int C = kAttnChunk;
    constexpr int DPL = D / 16;
    constexpr int PAIRS = (GMAX * D + kBlock - 1) / kBlock;   // (head, dim) pairs per thread
    constexpr int HSTEP = kBlock / D;                          // heads between a thread's pairs
    using T = ChunkTile<D>;
    auto& q_s = lds.q_s;
    auto& k_s = lds.k_s;
    auto& v_s = lds.v_s;
    auto& kc_s = lds.kc_s;
    auto& vc_s = lds.vc_s;
    auto& e_s = lds.e_s;
    auto& m_s = lds.m_s;
    auto& l_s = lds.l_s;
    auto& o_s = lds.o_s;

    const int g = bx;
    const int split = by;
    const int G = a.groups;
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid & (kWave - 1);

    int n, pos;
    if constexpr (STEP) {
        pos = *a.position;
        if (pos < 0 || pos >= a.capacity) {
            if (g == 0 && split == 0 && tid == 0) atomicOr(a.status, HQ_STEP_FULL);
            return 0;
        }
        n = pos + 1;
    } else {
        pos = -1;
        n = a.context + bz;     // query z of a batch sees z more positions
    }
    uint16_t* keys = a.keys;
    uint16_t* values = a.values;
    const float* qkv = a.qkv;
    bool rawq = STEP;     // q (and the current k/v) from the raw projection
    bool kvnew = STEP;    // the current position's k/v written and used from LDS
    if (!STEP && a.table) {
        // batched decode: query z is sequence z at its own position, in its
        // own cache (its layer slab: capacity * kv_heads * D elements)
        const int z = bz;
        const int zpos = *a.table->position[z];
        const int cap = a.table->capacity[z];
        n = min(max(zpos, 0), cap - 1) + 1;
        const size_t slab = size_t(cap) * size_t(a.kv_heads) * size_t(D);
        keys = a.table->keys[z] + size_t(a.layer) * slab;
        values = a.table->values[z] + size_t(a.layer) * slab;
        if (a.qkv) {
            // a batched step: row z of the raw projection, RoPE at the
            // (clamped) position; a position outside the cache (flagged by
            // the embedding kernel) writes nothing and reads the cache as is
            rawq = true;
            kvnew = zpos >= 0 && zpos < cap;
            pos = n - 1;
            qkv = a.qkv + size_t(z) * size_t(a.kv_heads) * size_t(G + 2) * D;
        }
    }
    const uint64_t* qll = nullptr;
    int32_t* zstatus = nullptr;
    if constexpr (QLL) {
        qll = a.qkv_ll + size_t(bz) * size_t(a.kv_heads) * size_t(G + 2) * D;
        zstatus = a.table->status[bz];
    }
    // dims lane and lane + 64 of raw-projection row `row`
    auto raw2 = [&](size_t row, float& x0, float& x1) {
        if constexpr (QLL) {
            poll_pair(qll + row * D + lane, ep, zstatus, x0, x1);
        } else {
            x0 = qkv[row * D + lane];
            x1 = qkv[row * D + lane + 64];
        }
    };
    // per-query regions of a batch (bz = 0 outside PLAIN batches)
    const size_t zq = size_t(bz) * size_t(a.kv_heads) * G * D;
    float* const out = a.out + zq;
    const int nc = (n + C - 1) / C;
    const int nsplit = (nc + CPB - 1) / CPB;
    if (split >= nsplit) return nsplit;
    const int c_begin = split * CPB;
    const int c_end = min(nc, c_begin + CPB);
    const size_t kv_off = size_t(g) * D;
    const int cur_chunk = kvnew ? nc - 1 : -1;    // chunk holding the current position

    uint4 kreg[T::kPerThread], vreg[T::kPerThread];
    {
        const int t0 = c_begin * C;
        load_chunk<D>(a, keys, values, t0, min(C, n - t0), c_begin == cur_chunk ? pos - t0 : -1, kv_off, kreg, vreg);
    }
    __builtin_amdgcn_sched_barrier(0);   // the chunk loads go out before the query prologue

    // ---- query heads (and from the raw projection the current k/v) ---------
    static_assert(!STEP || D == 128, "STEP mode is written for head_dim 128");
    bool plain_q = true;
    if constexpr (D == 128) if (rawq) {
        plain_q = false;
        const float* cs = a.rope_cos + size_t(pos) * (D / 2);
        const float* sn = a.rope_sin + size_t(pos) * (D / 2);
        for (int h = wave; h < G; h += kBlock / kWave) {
            float x0, x1;
            raw2(size_t(g * G + h), x0, x1);
            float p = __builtin_fmaf(x0, x0, 0.0f);
            p = __builtin_fmaf(x1, x1, p);
            const float ss = wave_tree_sum64_all(p);
            const float r = __builtin_sqrtf(ss / float(D) + a.eps);
            const float y0 = (x0 / r) * a.q_norm[lane];
            const float y1 = (x1 / r) * a.q_norm[lane + 64];
            const float c0 = cs[lane], s0 = sn[lane];
            q_s[h][lane] = y0 * c0 - y1 * s0;
            q_s[h][lane + 64] = y1 * c0 + y0 * s0;
        }
        if (kvnew && split == nsplit - 1) {
            const int heads = a.kv_heads * G;
            uint16_t* kdst = keys + size_t(pos) * a.time_stride + kv_off;
            uint16_t* vdst = values + size_t(pos) * a.time_stride + kv_off;
            if (wave == 0) {
                float x0, x1;
                raw2(size_t(heads + g), x0, x1);
                float p = __builtin_fmaf(x0, x0, 0.0f);
                p = __builtin_fmaf(x1, x1, p);
                const float ss = wave_tree_sum64_all(p);
                const float r = __builtin_sqrtf(ss / float(D) + a.eps);
                const float y0 = (x0 / r) * a.k_norm[lane];
                const float y1 = (x1 / r) * a.k_norm[lane + 64];
                const float c0 = cs[lane], s0 = sn[lane];
                const uint16_t h0 = f32_to_f16(y0 * c0 - y1 * s0);
                const uint16_t h1 = f32_to_f16(y1 * c0 + y0 * s0);
                kdst[lane] = h0;
                kdst[lane + 64] = h1;
                kc_s[lane] = h0;
                kc_s[lane + 64] = h1;
            } else if (wave == 1) {
                float x0, x1;
                raw2(size_t(heads + a.kv_heads + g), x0, x1);
                const uint16_t h0 = f32_to_f16(x0);
                const uint16_t h1 = f32_to_f16(x1);
                vdst[lane] = h0;
                vdst[lane + 64] = h1;
                vc_s[lane] = h0;
                vc_s[lane + 64] = h1;
            }
        } else if constexpr (QLL) {
            // a position outside the cache writes no K/V, but its rows'
            // entries are still awaited: this sequence's tail then starts
            // only after every qkv tile block of the launch has published,
            // i.e. has finished reading the q8/act rows the tail overwrites
            if (split == nsplit - 1 && wave < 2) {
                float x0, x1;
                raw2(size_t(a.kv_heads * G + wave * a.kv_heads + g), x0, x1);
            }
        }
    }
    if (plain_q)
        for (int i = tid; i < G * D; i += kBlock) q_s[i / D][i % D] = a.q[zq + size_t(g * G) * D + i];
    __syncthreads();

    const int grp = tid >> 4;       // 16 lane groups for the scores
    const int l16 = tid & 15;
    const float scale = 1.0f / __builtin_sqrtf(float(D));
    float qr[GMAX][DPL];
#pragma unroll
    for (int h = 0; h < GMAX; ++h)
#pragma unroll
        for (int j = 0; j < DPL; ++j) qr[h][j] = (h < G) ? q_s[h][l16 * DPL + j] : 0.0f;
    const int d = tid % D;
    const int h0 = tid / D;

    // the chunk loop stays rolled: one copy of its body keeps the kernel's
    // code small enough to stay resident in the instruction cache
#pragma unroll 1
    for (int ci = 0; ci < CPB; ++ci) {
        const int c = c_begin + ci;
        if (c >= c_end) break;
        const int t0 = c * C;
        const int tn = min(C, n - t0);

        // registers -> LDS (the current position's row comes from kc_s/vc_s)
#pragma unroll
        for (int r = 0; r < T::kPerThread; ++r) {
            const int id = tid + kBlock * r;
            const int t = id / T::kGroupsPerRow;
            const int d8 = id % T::kGroupsPerRow;
            if (id < T::kGroups && t < tn) {
                uint4 kv = kreg[r], vv = vreg[r];
                if (c == cur_chunk && t0 + t == pos) {
                    kv = *reinterpret_cast<const uint4*>(kc_s + d8 * 8);
                    vv = *reinterpret_cast<const uint4*>(vc_s + d8 * 8);
                }
                *reinterpret_cast<uint4*>(k_s + t * T::kRowHalves + d8 * 8) = kv;
                *reinterpret_cast<uint4*>(v_s + t * T::kRowHalves + d8 * 8) = vv;
            }
        }
        __syncthreads();
        if (c + 1 < c_end) {
            const int t1 = t0 + C;
            load_chunk<D>(a, keys, values, t1, min(C, n - t1), c + 1 == cur_chunk ? pos - t1 : -1, kv_off, kreg,
                          vreg);
        }
        __builtin_amdgcn_sched_barrier(0);

        // scores, 16 lanes per position
#pragma unroll
        for (int rep = 0; rep < C / 16; ++rep) {
            const int i = grp + 16 * rep;
            if (i < tn) {
                float k[DPL];
                const uint16_t* kr = k_s + i * T::kRowHalves + l16 * DPL;
#pragma unroll
                for (int j = 0; j < DPL; ++j) k[j] = f16_to_f32(kr[j]);
#pragma unroll
                for (int h = 0; h < GMAX; ++h) {
                    if (h < G) {
                        float pp = 0.0f;
#pragma unroll
                        for (int j = 0; j < DPL; ++j) pp = __builtin_fmaf(qr[h][j], k[j], pp);
                        const float dot = row_tree_sum16(pp);
                        if (l16 == 0) e_s[h][i] = dot * scale;
                    }
                }
            } else if (l16 == 0) {
#pragma unroll
                for (int h = 0; h < GMAX; ++h)
                    if (h < G) e_s[h][i] = -__builtin_inff();
            }
        }
        __syncthreads();

        // chunk softmax statistics, one wave per head
        for (int h = wave; h < G; h += kBlock / kWave) {
            const float sc = e_s[h][lane];
            const float m = wave_max64_all(sc);
            const float e = (lane < tn) ? spec_expf(sc - m) : 0.0f;
            const float l = wave_tree_sum64(e);
            e_s[h][lane] = e;
            if (lane == 0) { m_s[h][ci] = m; l_s[h][ci] = l; }
        }
        __syncthreads();

        // partial V accumulation from LDS: an fmaf chain over ascending
        // positions; the LDS reads of 8 positions are issued before their
        // fmas so their latency is paid once per 8 positions
        float o_acc[PAIRS];
#pragma unroll
        for (int r = 0; r < PAIRS; ++r) o_acc[r] = 0.0f;
        int i = 0;
        for (; i + 8 <= tn; i += 8) {
            float v[8], e[PAIRS][8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                v[j] = f16_to_f32(v_s[(i + j) * T::kRowHalves + d]);
#pragma unroll
                for (int r = 0; r < PAIRS; ++r) {
                    const int h = min(h0 + HSTEP * r, GMAX - 1);
                    e[r][j] = e_s[h][i + j];
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int r = 0; r < PAIRS; ++r)
                    o_acc[r] = __builtin_fmaf(e[r][j], v[j], o_acc[r]);
        }
        for (; i < tn; ++i) {
            const float v = f16_to_f32(v_s[i * T::kRowHalves + d]);
#pragma unroll
            for (int r = 0; r < PAIRS; ++r) {
                const int h = min(h0 + HSTEP * r, GMAX - 1);
                o_acc[r] = __builtin_fmaf(e_s[h][i], v, o_acc[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < PAIRS; ++r) {
            const int h = h0 + HSTEP * r;
            if (h < G) o_s[ci][h][d] = o_acc[r];
        }
        __syncthreads();
    }

    const int pstride = D + 2;
    const int nmine = c_end - c_begin;
    if (nsplit == 1) {
        // every chunk is in this block: combine in ascending chunk order
#pragma unroll
        for (int r = 0; r < PAIRS; ++r) {
            const int h = h0 + HSTEP * r;
            if (h >= G) continue;
            float M = -__builtin_inff();
            for (int ci = 0; ci < nmine; ++ci) M = fmaxf(M, m_s[h][ci]);
            float L = 0.0f, O = 0.0f;
            for (int ci = 0; ci < nmine; ++ci) {
                const float al = spec_expf(m_s[h][ci] - M);
                L = __builtin_fmaf(al, l_s[h][ci], L);
                O = __builtin_fmaf(al, o_s[ci][h][d], O);
            }
            if constexpr (TAILS) tail_store(a.ll_out + zq + size_t(g * G + h) * D + d, O * (1.0f / L), ep);
            else out[size_t(g * G + h) * D + d] = O * (1.0f / L);
        }
        return nsplit;
    }

    // several splits: publish this block's chunk partials
    for (int ci = 0; ci < nmine; ++ci) {
        const int c = c_begin + ci;
#pragma unroll
        for (int r = 0; r < PAIRS; ++r) {
            const int h = h0 + HSTEP * r;
            if (h >= G) continue;
            const size_t off = size_t(bz) * size_t(a.kv_heads) * G * a.max_chunks * pstride +
                               (size_t(g * G + h) * a.max_chunks + c) * pstride;
            if constexpr (TAILS) {
                uint64_t* pp = a.ll_part + off;
                tail_store(pp + 2 + d, o_s[ci][h][d], ep);
                if (d == 0) { tail_store(pp, m_s[h][ci], ep); tail_store(pp + 1, l_s[h][ci], ep); }
            } else {
                float* pp = a.part + off;
                publish_f(pp + 2 + d, o_s[ci][h][d]);
                if (d == 0) { publish_f(pp, m_s[h][ci]); publish_f(pp + 1, l_s[h][ci]); }
            }
        }
    }
    // (attention_combine_kernel or batch_combine_quant_kernel, launched next
    // on the stream, or this launch's tail combines them)
    return nsplit;
}

// Tail of a batched-step attention launch (TAILS): block (sequence s, part
// qt) finishes heads [qt*HQ, qt*HQ + HQ) of sequence s (HQ = H/8, two heads
// per pass of 256 threads, NO outputs per thread): each output is
// the single split's entry, or the combine of the chunk partials exactly as
// batch_combine_quant_kernel computes it (M = max of m_c; a_c = exp(m_c -
// M); L and O fmaf chains over ascending c; out = O * (1 / L)).  The row's
// maximum |out| is each part's maximum (order-free) handed between the
// eight blocks as entries (they wait for each other: the launch's other
// blocks wait for nobody, so they finish and the at most 8 * 32 tail blocks
// all get a place on the chip); then the same quantization (amax floored at 1e-5,
// quant_i8 with 127 / amax, de-interleaved, act = amax / 127).
constexpr int kAttnTailChunks = 8;   // chunks per combine batch (more take several batches)
constexpr int kAttnMaxSplits = 8;    // splits (blockIdx.y) in a batched step's attention grid
constexpr int kAttnTailParts = 8;    // tail blocks per sequence
constexpr int kAttnTailNO = 2;       // outputs per thread: up to 2 * 2 * 8 = 32 query heads
template <int D, bool BIG>
__device__ void attention_tail(const AttnParams& a, int s, int qt, uint32_t ep)
{
    static_assert(D == kBlock / 2, "two heads per pass of the block");
    constexpr int NO = kAttnTailNO;
    constexpr int NC = kAttnTailChunks;
    constexpr int pstride = D + 2;
    __shared__ float ml_s[2 * NO][NC][2];
    __shared__ float wmax_s[kBlock / kWave];
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int d = tid % D, h0 = tid / D;
    const int H = a.kv_heads * a.groups;
    const int HQ = H / kAttnTailParts;
    const int hb = qt * HQ;
    const int cap = a.table->capacity[s];
    const int n = min(max(*a.table->position[s], 0), cap - 1) + 1;
    const int nc = (n + kAttnChunk - 1) / kAttnChunk;
    const uint64_t ready = uint64_t(ep) << 32;
    const size_t HD = size_t(H) * D;
    int32_t* status = a.table->status[s];
    float val[NO];
    auto wait = [&](auto& e, auto&& reload) {
        unsigned spins = 0;
        while (true) {
            bool pending = false;
            unrolled<sizeof(e) / sizeof(e[0])>([&](auto j) { pending |= !tail_ready(e[j], ep); });
            if (!pending) return;
            if (++spins == kTailSpinLimit) {
                atomicOr(status, HQ_STEP_SYNC);
                return;
            }
            __builtin_amdgcn_s_sleep(1);
            unrolled<sizeof(e) / sizeof(e[0])>([&](auto j) {
                if (!tail_ready(e[j], ep)) e[j] = reload(j);
            });
        }
    };
    if (nc <= a.cpb) {
        // one split held every chunk of each head and combined them itself
        uint64_t e[NO];
        auto src = [&](auto i) { return a.ll_out + size_t(s) * HD + size_t(hb + h0 + 2 * i) * D + d; };
        unrolled<NO>([&](auto i) { e[i] = h0 + 2 * i < HQ ? tail_load(src(i)) : ready; });
        wait(e, [&](auto i) { return tail_load(src(i)); });
        unrolled<NO>([&](auto i) { val[i] = h0 + 2 * i < HQ ? bits_f32(uint32_t(e[i])) : 0.0f; });
    } else if constexpr (!BIG) {
        // every context within NC chunks (the launch checked max_chunks):
        // one batch, straight-line code
        const uint64_t* base = a.ll_part + size_t(s) * size_t(H) * a.max_chunks * pstride;
        // m_c and l_c of the part's heads: entry tid = (head, chunk, m|l)
        {
            uint64_t e[1];
            const int hq = tid / (2 * NC), c = (tid / 2) % NC, kind = tid & 1;
            const bool mine = hq < HQ && c < nc;
            auto src = [&](auto) { return base + (size_t(hb + hq) * a.max_chunks + c) * pstride + kind; };
            e[0] = mine ? tail_load(src(0)) : ready;
            wait(e, [&](auto j) { return tail_load(src(j)); });
            if (mine) ml_s[hq][c][kind] = bits_f32(uint32_t(e[0]));
        }
        // o_c[d] of this thread's heads
        uint64_t o[NO * NC];
        auto osrc = [&](auto j) {
            const int i = int(j) / NC, c = int(j) % NC;
            return base + (size_t(hb + h0 + 2 * i) * a.max_chunks + c) * pstride + 2 + d;
        };
        unrolled<NO * NC>([&](auto j) {
            o[j] = (h0 + 2 * (int(j) / NC) < HQ && int(j) % NC < nc) ? tail_load(osrc(j)) : ready;
        });
        wait(o, [&](auto j) { return tail_load(osrc(j)); });
        __syncthreads();   // ml_s
        unrolled<NO>([&](auto i) {
            const int hq = h0 + 2 * i;
            if (hq < HQ) {
                float M = ml_s[hq][0][0];
                for (int c = 1; c < nc; ++c) M = fmaxf(M, ml_s[hq][c][0]);
                float L = 0.0f, O = 0.0f;
                unrolled<NC>([&](auto c) {
                    if (c < nc) {
                        const float al = spec_expf(ml_s[hq][c][0] - M);
                        L = __builtin_fmaf(al, ml_s[hq][c][1], L);
                        O = __builtin_fmaf(al, bits_f32(uint32_t(o[i * NC + c])), O);
                    }
                });
                val[i] = O * (1.0f / L);
            } else {
                val[i] = 0.0f;
            }
        });
    } else {
        const uint64_t* base = a.ll_part + size_t(s) * size_t(H) * a.max_chunks * pstride;
        // m_c (and l_c) of the part's heads for chunks [cb, cb + NC):
        // entry tid = (head, chunk, m|l), into ml_s
        auto load_ml = [&](int cb, bool with_l) {
            uint64_t e[1];
            const int hq = tid / (2 * NC), c = cb + (tid / 2) % NC, kind = tid & 1;
            const bool mine = hq < HQ && c < nc && (with_l || kind == 0);
            auto src = [&](auto) { return base + (size_t(hb + hq) * a.max_chunks + c) * pstride + kind; };
            e[0] = mine ? tail_load(src(0)) : ready;
            wait(e, [&](auto j) { return tail_load(src(j)); });
            if (mine) ml_s[hq][c - cb][kind] = bits_f32(uint32_t(e[0]));
        };
        // o_c[d] of this thread's heads for chunks [cb, cb + NC)
        uint64_t o[NO * NC];
        auto load_o = [&](int cb) {
            auto osrc = [&](auto j) {
                const int i = int(j) / NC, c = cb + int(j) % NC;
                return base + (size_t(hb + h0 + 2 * i) * a.max_chunks + c) * pstride + 2 + d;
            };
            unrolled<NO * NC>([&](auto j) {
                o[j] = (h0 + 2 * (int(j) / NC) < HQ && cb + int(j) % NC < nc) ? tail_load(osrc(j)) : ready;
            });
            wait(o, [&](auto j) { return tail_load(osrc(j)); });
        };
        // M = m_0, then fmaxf with m_1, m_2, ... (a first pass over every
        // batch of NC chunks when there are more); then the L and O chains
        // over ascending chunks, batch by batch
        float M[NO], L[NO], O[NO];
        unrolled<NO>([&](auto i) { L[i] = 0.0f; O[i] = 0.0f; });
        if (nc > NC) {
            for (int cb = 0; cb < nc; cb += NC) {
                load_ml(cb, false);
                __syncthreads();   // ml_s
                unrolled<NO>([&](auto i) {
                    const int hq = h0 + 2 * i;
                    if (hq < HQ)
                        for (int c = 0; c < min(NC, nc - cb); ++c)
                            M[i] = cb + c == 0 ? ml_s[hq][0][0] : fmaxf(M[i], ml_s[hq][c][0]);
                });
                __syncthreads();   // ml_s is written again
            }
        }
        for (int cb = 0; cb < nc; cb += NC) {
            load_ml(cb, true);
            load_o(cb);
            __syncthreads();   // ml_s
            unrolled<NO>([&](auto i) {
                const int hq = h0 + 2 * i;
                if (hq < HQ) {
                    if (nc <= NC) {
                        M[i] = ml_s[hq][0][0];
                        for (int c = 1; c < nc; ++c) M[i] = fmaxf(M[i], ml_s[hq][c][0]);
                    }
                    unrolled<NC>([&](auto c) {
                        if (cb + c < nc) {
                            const float al = spec_expf(ml_s[hq][c][0] - M[i]);
                            L[i] = __builtin_fmaf(al, ml_s[hq][c][1], L[i]);
                            O[i] = __builtin_fmaf(al, bits_f32(uint32_t(o[i * NC + c])), O[i]);
                        }
                    });
                }
            });
            __syncthreads();   // ml_s is written again
        }
        unrolled<NO>([&](auto i) { val[i] = h0 + 2 * i < HQ ? O[i] * (1.0f / L[i]) : 0.0f; });
    }
    // the row's maximum: this part's, then the eight parts'
    float mx = 0.0f;
    unrolled<NO>([&](auto i) { mx = fmaxf(mx, fabsf(val[i])); });
    mx = wave_max64_all(mx);
    if (lane == 0) wmax_s[tid / kWave] = mx;
    __syncthreads();
    if (tid == 0) {
        float qm = wmax_s[0];
        for (int w = 1; w < kBlock / kWave; ++w) qm = fmaxf(qm, wmax_s[w]);
        tail_store(a.ll_max + size_t(s) * kAttnTailParts + qt, qm, ep);
    }
    // lane q < 8 of wave 0 waits for part q's maximum (one poll per part
    // and round: polled by every thread, the 2048 reads of each entry per
    // round held the exchange back), then the block reads it from LDS
    __shared__ float amax_s;
    if (tid < kWave) {
        const bool mine = lane < kAttnTailParts;
        const uint64_t* mrow = a.ll_max + size_t(s) * kAttnTailParts;
        uint64_t e = mine ? tail_load(mrow + lane) : uint64_t(ep) << 32;
        unsigned spins = 0;
        while (__builtin_amdgcn_ballot_w64(!tail_ready(e, ep))) {   // (wave-uniform)
            if (++spins == kTailSpinLimit) {
                if (lane == 0) atomicOr(status, HQ_STEP_SYNC);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
            if (!tail_ready(e, ep)) e = tail_load(mrow + lane);
        }
        const float am = wave_max64_all(mine ? bits_f32(uint32_t(e)) : 0.0f);   // (order-free)
        if (lane == 0) amax_s = fmaxf(am, 1e-5f);
    }
    __syncthreads();
    const float amax = amax_s;
    const float inv = 127.0f / amax;
    unrolled<NO>([&](auto i) {
        if (h0 + 2 * i < HQ) a.q8[bq_pos(s, xq_offset((hb + h0 + 2 * i) * D + d), a.kp)] = quant_i8(val[i], inv);
    });
    if (qt == 0 && tid == 0) a.act[s] = amax / 127.0f;
}

// BIG: the batched step's launch for states of more than kAttnTailChunks
// chunks (a separate instantiation: the split walk and the batched tail
// combine take registers that the common case would pay for in occupancy).
template <int D, int GMAX, bool STEP, int CPB, bool TAILS = false, bool BIG = false>
__global__ __launch_bounds__(kBlock) void attention_kernel(AttnParams a)
{
    __shared__ AttnLds<D, GMAX, CPB> lds;
    const uint32_t ep = TAILS ? (*a.epoch_ctr << 8) | uint32_t(a.epoch_id) : 0u;
    if constexpr (BIG) {
        // splits y, y + gridDim.y, ... of the query (the grid holds fewer
        // splits than the largest capacity allows: blocks walk the rest,
        // and splits past a context exit at once)
        for (int y = int(blockIdx.y);;) {
            const int nsplit =
                attention_block<D, GMAX, STEP, CPB, TAILS>(a, ep, lds, int(blockIdx.x), y, int(blockIdx.z));
            y += int(gridDim.y);
            if (y >= nsplit) break;   // (block-uniform)
            __syncthreads();          // the block's LDS is filled again
        }
    } else {
        attention_block<D, GMAX, STEP, CPB, TAILS>(a, ep, lds, int(blockIdx.x), int(blockIdx.y), int(blockIdx.z));
    }
    if constexpr (TAILS) {
        const int lin = int(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z));
        const int u = lin - int(gridDim.x * gridDim.y * gridDim.z) + kAttnTailParts * a.batch;
        if (u >= 0) attention_tail<D, BIG>(a, u % a.batch, u / a.batch, ep);   // (block-uniform)
    }
}

// The batched step's qkv GEMM and attention in one launch: blocks [0, tiles)
// compute the qkv rows (gemm_lds_block, K up to 2560) into {value, epoch}
// entries; the blocks after them are the attention launch's blocks (kv head,
// split, sequence; gy splits) with their tails, and take the raw projection
// from those entries.  Every block an attention block waits for has started
// before it (blocks start in index order).  One LDS buffer serves either role.
template <int RG, int BT, int CPB, bool BIG>
__global__ __launch_bounds__(kBlock) void qkv_attention_kernel(GemmParams gp, AttnParams a, int tiles, int gy)
{
    constexpr int HMAX = 1280;
    constexpr int R = 16 * RG;
    constexpr int DS = (2 * HMAX / 128 + 3) / 4;
    constexpr int CPT = (R * HMAX / 16 + kBlock - 1) / kBlock;
    union Lds {
        alignas(16) uint8_t gemm[R * (HMAX + 16)];
        AttnLds<128, 4, CPB> at;
    };
    __shared__ Lds lds;
    if (int(blockIdx.x) < tiles) {   // (block-uniform)
        gemm_lds_block<RG, 4, BT, DS, CPT, HMAX, false, -1>(gp, lds.gemm);
        return;
    }
    const uint32_t ep = (*a.epoch_ctr << 8) | uint32_t(a.epoch_id);
    const int k = int(blockIdx.x) - tiles;
    const int gx = a.kv_heads;
    if constexpr (BIG) {
        for (int y = (k / gx) % gy;;) {
            const int nsplit =
                attention_block<128, 4, false, CPB, true, true>(a, ep, lds.at, k % gx, y, k / (gx * gy));
            y += gy;
            if (y >= nsplit) break;   // (block-uniform)
            __syncthreads();          // the block's LDS is filled again
        }
    } else {
        attention_block<128, 4, false, CPB, true, true>(a, ep, lds.at, k % gx, (k / gx) % gy, k / (gx * gy));
    }
    const int u = k - gx * gy * a.batch + kAttnTailParts * a.batch;
    if (u >= 0) attention_tail<128, BIG>(a, u % a.batch, u / a.batch, ep);   // (block-uniform)
}

// ---- batched step attention, one block per (sequence, kv head) -------------------
//
// For batches of more than 8 sequences whose states hold at most kSeqChunks
// chunks: block (z, g) of 1024 threads runs kv head g of sequence z over its
// whole context, four 256-thread groups side by side (group u takes chunks u,
// u + 4), each chunk exactly as attention_block computes it (the group's K/V
// loads go out one chunk ahead, into registers, then LDS; scores, chunk
// statistics, V chains).  The chunk partials stay in the block's LDS, and
// threads (head, dim) combine them over ascending chunks as the split
// launches' tails do (M = m_0, then fmaxf with m_1, ...; a_c = exp(m_c - M);
// L and O fmaf chains; out = O * (1 / L)).  The row's maximum |out| is
// exchanged among the sequence's eight kv-head blocks as {value, epoch}
// entries (bounded waits, HQ_STEP_SYNC), and each block quantizes its four
// heads into the o GEMM's input row (amax floored at 1e-5, quant_i8 with 127
// / amax, de-interleaved, act = amax / 127).  No chunk partial leaves the
// CU, and no tail block waits for a place on the chip.
constexpr int kSeqSubs = 4;                        // 256-thread groups per block
constexpr int kSeqThreads = kSeqSubs * kBlock;
constexpr int kSeqChunks = 8;                      // contexts of up to 8 chunks
#ifndef HQ_SEQ_MIN_BATCH
#define HQ_SEQ_MIN_BATCH 9
#endif
constexpr int kSeqMinBatch = HQ_SEQ_MIN_BATCH;     // batches that take seq_attention_kernel

struct SeqAttnLds {
    float q_s[4][128];
    uint16_t kc_s[128];
    uint16_t vc_s[128];
    struct Sub {
        alignas(16) uint16_t k_s[kAttnChunk * ChunkTile<128>::kRowHalves];
        alignas(16) uint16_t v_s[kAttnChunk * ChunkTile<128>::kRowHalves];
        float e_s[4][kAttnChunk];
    } sub[kSeqSubs];
    float m_s[4][kSeqChunks];
    float l_s[4][kSeqChunks];
    float al_s[4][kSeqChunks];
    float o_s[kSeqChunks][4][128];
    float wmax[kSeqThreads / kWave];
    float amax;
};

__global__ __launch_bounds__(kSeqThreads) void seq_attention_kernel(AttnParams a)
{
    constexpr int D = 128, G = 4, C = kAttnChunk, DPL = D / 16;
    using T = ChunkTile<D>;
    __shared__ SeqAttnLds S;
    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid & (kWave - 1);
    const int sub = tid / kBlock, st = tid % kBlock, sw = wave % (kBlock / kWave);
    const int g = int(blockIdx.x) % a.kv_heads, z = int(blockIdx.x) / a.kv_heads;
    const uint32_t ep = (*a.epoch_ctr << 8) | uint32_t(a.epoch_id);
    int32_t* status = a.table->status[z];
    // sequence z at its own position, in its own cache; a position outside
    // the cache writes nothing and reads the cache as is
    const int zpos = *a.table->position[z];
    const int cap = a.table->capacity[z];
    const int n = min(max(zpos, 0), cap - 1) + 1;
    const bool kvnew = zpos >= 0 && zpos < cap;
    const int pos = n - 1;
    const size_t slab = size_t(cap) * size_t(a.kv_heads) * size_t(D);
    uint16_t* keys = a.table->keys[z] + size_t(a.layer) * slab;
    uint16_t* values = a.table->values[z] + size_t(a.layer) * slab;
    const float* qkv = a.qkv + size_t(z) * size_t(a.kv_heads) * size_t(G + 2) * D;
    const int nc = (n + C - 1) / C;               // <= kSeqChunks (checked by the launch)
    const int cur_chunk = kvnew ? nc - 1 : -1;    // chunk holding the current position
    const size_t kv_off = size_t(g) * D;

    // a chunk's K loads go out before its V loads (a wave's loads complete
    // in issue order); they are buffer loads, all issued on every path, so
    // the compiler's waits count exactly the loads behind each use
    uint4 kreg[T::kPerThread], vreg[T::kPerThread];
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    const __amdgpu_buffer_rsrc_t rk = raw_rsrc(keys, int(slab * 2));
    const __amdgpu_buffer_rsrc_t rv = raw_rsrc(values, int(slab * 2));
    // (a row outside the chunk, or a chunk past the context: an offset past
    // the buffer, read as 0 without a memory access)
    auto offsets = [&](int c, uint32_t (&vo)[T::kPerThread]) {
        const int t0 = c * C;
        const int tn = min(C, n - t0);   // (<= 0 past the context)
        const int skip_t = c == cur_chunk ? pos - t0 : -1;
#pragma unroll
        for (int r = 0; r < T::kPerThread; ++r) {
            const int id = st + kBlock * r;
            const int t = id / T::kGroupsPerRow;
            const int d8 = id % T::kGroupsPerRow;
            const bool ok = id < T::kGroups && t < tn && t != skip_t;
            vo[r] = ok ? uint32_t((size_t(t0 + t) * a.time_stride + kv_off + size_t(d8) * 8) * 2) : 0x80000000u;
        }
    };
    auto load_m = [&](const __amdgpu_buffer_rsrc_t& rs, const uint32_t (&vo)[T::kPerThread], uint4 (&reg)[T::kPerThread]) {
#pragma unroll
        for (int r = 0; r < T::kPerThread; ++r) {
            const v4u w = __builtin_amdgcn_raw_buffer_load_b128(rs, vo[r], 0, 0);
            reg[r] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    };
    // registers -> LDS for one matrix (the current position's row comes
    // from kc_s / vc_s)
    auto to_lds = [&](int c, int tn, const uint4 (&reg)[T::kPerThread], const uint16_t* cur, uint16_t* dst) {
#pragma unroll
        for (int r = 0; r < T::kPerThread; ++r) {
            const int id = st + kBlock * r;
            const int t = id / T::kGroupsPerRow;
            const int d8 = id % T::kGroupsPerRow;
            if (id < T::kGroups && t < tn) {
                uint4 w = reg[r];
                if (c == cur_chunk && c * C + t == pos) w = *reinterpret_cast<const uint4*>(cur + d8 * 8);
                *reinterpret_cast<uint4*>(dst + t * T::kRowHalves + d8 * 8) = w;
            }
        }
    };
    // ---- query heads and the current position's k/v ----------------------
    // Every wave loads its operands first (waves 0-3 query head `wave`, wave
    // 4 the k row, wave 5 the v row, the others query head 0 unused), then
    // its group's first chunk; every load is issued on every path, so the
    // waits the compiler places count exactly the loads behind each use.
    const int heads = a.kv_heads * G;
    const int prow = wave < G ? g * G + wave : wave == G ? heads + g : wave == G + 1 ? heads + a.kv_heads + g : g * G;
    const float x0 = qkv[size_t(prow) * D + lane];
    const float x1 = qkv[size_t(prow) * D + lane + 64];
    const float* nw = wave == G ? a.k_norm : a.q_norm;
    const float nw0 = nw[lane], nw1 = nw[lane + 64];
    const float c0 = a.rope_cos[size_t(pos) * (D / 2) + lane];
    const float s0 = a.rope_sin[size_t(pos) * (D / 2) + lane];
    // Only the first chunk's K rows go out now.  A wave whose loads find the
    // CU's memory pipe full stalls at the load instruction, so a wave that
    // issued its V rows as well would reach its next computation only once
    // most of the launch's K/V bytes had arrived; the V rows go out once
    // the K rows are in LDS, and the scores run while they stream.
    uint32_t vo[T::kPerThread];
    offsets(sub, vo);
    load_m(rk, vo, kreg);
    if (wave <= G) {
        float p = __builtin_fmaf(x0, x0, 0.0f);
        p = __builtin_fmaf(x1, x1, p);
        const float ss = wave_tree_sum64_all(p);
        const float r = __builtin_sqrtf(ss / float(D) + a.eps);
        const float y0 = (x0 / r) * nw0;
        const float y1 = (x1 / r) * nw1;
        const float r0 = y0 * c0 - y1 * s0;
        const float r1 = y1 * c0 + y0 * s0;
        if (wave < G) {
            S.q_s[wave][lane] = r0;
            S.q_s[wave][lane + 64] = r1;
        } else if (kvnew) {
            const uint16_t h0 = f32_to_f16(r0);
            const uint16_t h1 = f32_to_f16(r1);
            // (buffer stores: flat ones would make the compiler's waits
            // for the chunk loads conservative)
            const uint32_t o = uint32_t((size_t(pos) * a.time_stride + kv_off + lane) * 2);
            __builtin_amdgcn_raw_buffer_store_b16(h0, rk, o, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b16(h1, rk, o + 128, 0, 0);
            S.kc_s[lane] = h0;
            S.kc_s[lane + 64] = h1;
        }
    } else if (wave == G + 1 && kvnew) {
        const uint16_t h0 = f32_to_f16(x0);
        const uint16_t h1 = f32_to_f16(x1);
        const uint32_t o = uint32_t((size_t(pos) * a.time_stride + kv_off + lane) * 2);
        __builtin_amdgcn_raw_buffer_store_b16(h0, rv, o, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b16(h1, rv, o + 128, 0, 0);
        S.vc_s[lane] = h0;
        S.vc_s[lane + 64] = h1;
    }
    lds_sync();

    const int grp = st >> 4;        // 16 lane groups for the scores
    const int l16 = st & 15;
    const float scale = 1.0f / __builtin_sqrtf(float(D));
    float qr[G][DPL];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int j = 0; j < DPL; ++j) qr[h][j] = S.q_s[h][l16 * DPL + j];
    const int d = st % D;
    const int h0 = st / D;          // V chains: heads h0 and h0 + 2
    auto& B = S.sub[sub];
    const int rounds = (nc + kSeqSubs - 1) / kSeqSubs;

    // every group passes the same barriers, with or without a chunk; the
    // barriers order LDS only (lds_sync), so loads in flight stay in flight
#pragma unroll 1
    for (int rd = 0; rd < rounds; ++rd) {
        const int c = sub + kSeqSubs * rd;
        const bool mine = c < nc;   // (group-uniform)
        const int t0 = c * C;
        const int tn = mine ? min(C, n - t0) : 0;
        if (mine) to_lds(c, tn, kreg, S.kc_s, B.k_s);
        load_m(rv, vo, vreg);   // this chunk's V rows
        lds_sync();
        if (mine) {
            // scores, 16 lanes per position
#pragma unroll
            for (int rep = 0; rep < C / 16; ++rep) {
                const int i = grp + 16 * rep;
                if (i < tn) {
                    float k[DPL];
                    const uint16_t* kr = B.k_s + i * T::kRowHalves + l16 * DPL;
#pragma unroll
                    for (int j = 0; j < DPL; ++j) k[j] = f16_to_f32(kr[j]);
#pragma unroll
                    for (int h = 0; h < G; ++h) {
                        float pp = 0.0f;
#pragma unroll
                        for (int j = 0; j < DPL; ++j) pp = __builtin_fmaf(qr[h][j], k[j], pp);
                        const float dot = row_tree_sum16(pp);
                        if (l16 == 0) B.e_s[h][i] = dot * scale;
                    }
                } else if (l16 == 0) {
#pragma unroll
                    for (int h = 0; h < G; ++h) B.e_s[h][i] = -__builtin_inff();
                }
            }
        }
        if (mine) to_lds(c, tn, vreg, S.vc_s, B.v_s);
        offsets(c + kSeqSubs, vo);   // the group's next chunk (past the context: nothing)
        load_m(rk, vo, kreg);
        lds_sync();
        if (mine) {
            // chunk softmax statistics, one wave of the group per head
            const int h = sw;
            const float sc = B.e_s[h][lane];
            const float m = wave_max64_all(sc);
            const float e = (lane < tn) ? spec_expf(sc - m) : 0.0f;
            const float l = wave_tree_sum64(e);
            B.e_s[h][lane] = e;
            if (lane == 0) { S.m_s[h][c] = m; S.l_s[h][c] = l; }
        }
        lds_sync();
        if (mine) {
            // V chains over ascending positions, eight LDS reads ahead
            float o_acc[2] = {0.0f, 0.0f};
            int i = 0;
            for (; i + 8 <= tn; i += 8) {
                float v[8], e[2][8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    v[j] = f16_to_f32(B.v_s[(i + j) * T::kRowHalves + d]);
#pragma unroll
                    for (int r = 0; r < 2; ++r) e[r][j] = B.e_s[h0 + 2 * r][i + j];
                }
#pragma unroll
                for (int j = 0; j < 8; ++j)
#pragma unroll
                    for (int r = 0; r < 2; ++r) o_acc[r] = __builtin_fmaf(e[r][j], v[j], o_acc[r]);
            }
            for (; i < tn; ++i) {
                const float v = f16_to_f32(B.v_s[i * T::kRowHalves + d]);
#pragma unroll
                for (int r = 0; r < 2; ++r) o_acc[r] = __builtin_fmaf(B.e_s[h0 + 2 * r][i], v, o_acc[r]);
            }
#pragma unroll
            for (int r = 0; r < 2; ++r) S.o_s[c][h0 + 2 * r][d] = o_acc[r];
        }
        lds_sync();
    }

    // ---- combine over ascending chunks, thread (head, dim) -----------------
    // (a_c once per (head, chunk): thread h * 8 + c)
    if (tid < G * kSeqChunks) {
        const int h = tid / kSeqChunks, c = tid % kSeqChunks;
        float M = S.m_s[h][0];
        for (int j = 1; j < nc; ++j) M = fmaxf(M, S.m_s[h][j]);
        if (c < nc) S.al_s[h][c] = spec_expf(S.m_s[h][c] - M);
    }
    lds_sync();
    float val = 0.0f;
    if (tid < G * D) {
        const int h = tid / D, dd = tid % D;
        float L = 0.0f, O = 0.0f;
        for (int c = 0; c < nc; ++c) {
            const float al = S.al_s[h][c];
            L = __builtin_fmaf(al, S.l_s[h][c], L);
            O = __builtin_fmaf(al, S.o_s[c][h][dd], O);
        }
        val = O * (1.0f / L);
    }
    // ---- the row's maximum over the sequence's kv-head blocks, then quant --
    float mx = wave_max64_all(fabsf(val));   // (threads past G * D hold 0)
    if (lane == 0) S.wmax[wave] = mx;
    lds_sync();
    if (wave == 0) {
        uint64_t* mrow = a.ll_max + size_t(z) * kAttnTailParts;
        if (lane == 0) {
            float qm = S.wmax[0];
            for (int w = 1; w < kSeqThreads / kWave; ++w) qm = fmaxf(qm, S.wmax[w]);
            tail_store(mrow + g, qm, ep);
        }
        // lane q < 8 waits for block q's maximum
        const bool mine = lane < kAttnTailParts;
        uint64_t e = mine ? tail_load(mrow + lane) : (uint64_t(ep) << 32);
        unsigned spins = 0;
        while (__builtin_amdgcn_ballot_w64(!tail_ready(e, ep))) {   // (wave-uniform)
            if (++spins == kTailSpinLimit) {
                if (lane == 0) atomicOr(status, HQ_STEP_SYNC);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
            if (!tail_ready(e, ep)) e = tail_load(mrow + lane);
        }
        float am = mine ? bits_f32(uint32_t(e)) : 0.0f;
        am = wave_max64_all(am);
        if (lane == 0) S.amax = fmaxf(am, 1e-5f);
    }
    lds_sync();
    const float amax = S.amax;
    const float inv = 127.0f / amax;
    if (tid < G * D) a.q8[bq_pos(z, xq_offset(g * G * D + tid), a.kp)] = quant_i8(val, inv);
    if (g == 0 && tid == 0) a.act[z] = amax / 127.0f;
}


// Combine of the chunk partials when a context spans several chunks: thread
// (blockIdx.x * kBlock + tid) is output element (query head hh, dim d) of
// query z = blockIdx.y.  Same arithmetic as the single-chunk combine above:
// M = max_c m_c; a_c = exp(m_c - M); L and O as fmaf chains over ascending
// c; out = O * (1 / L).  The block's heads' m_c and l_c are staged in LDS
// (batches of CB chunks), the a_c computed once per chunk in place of m_c,
// and the o values read 64 chunks at a time (coalesced over d).
template <int D, bool STEP>
__global__ __launch_bounds__(kBlock) void attention_combine_kernel(AttnParams a)
{
    constexpr int C = kAttnChunk;
    constexpr int HPB = kBlock / D;           // query heads per block
    constexpr int CB = 4096 / HPB;            // chunks per staged batch
    constexpr int OB = 64;                    // o values in flight per thread
    __shared__ float m_s[HPB][CB];
    __shared__ float l_s[HPB][CB];
    __shared__ float red_s[kBlock];
    const int z = blockIdx.y;
    int n;
    if constexpr (STEP) {
        const int pos = *a.position;
        if (pos < 0 || pos >= a.capacity) return;   // (flagged by attention_kernel)
        n = pos + 1;
    } else if (a.table) {
        const int zpos = *a.table->position[z];
        n = min(max(zpos, 0), a.table->capacity[z] - 1) + 1;
    } else {
        n = a.context + z;
    }
    const int nc = (n + C - 1) / C;
    if (nc <= 1) return;                       // attention_kernel combined it in-block
    const int heads = a.kv_heads * a.groups;
    const int tid = threadIdx.x;
    const int hl = tid / D, d = tid % D;
    const int hh = blockIdx.x * HPB + hl;
    const bool live = hh < heads;
    constexpr int pstride = D + 2;
    const float* part = a.part + size_t(z) * size_t(heads) * a.max_chunks * pstride;
    const float* ph = part + size_t(min(hh, heads - 1)) * a.max_chunks * pstride;

    float M = -__builtin_inff();
    if (nc > CB) {
        // M from every chunk first (several staged batches follow)
        float mm = -__builtin_inff();
        for (int c = d; c < nc; c += D) mm = fmaxf(mm, read_f(ph + size_t(c) * pstride));
        red_s[tid] = mm;
        __syncthreads();
        for (int i = 0; i < D; ++i) M = fmaxf(M, red_s[hl * D + i]);
    }
    float L = 0.0f, O = 0.0f;
    for (int c0 = 0; c0 < nc; c0 += CB) {
        const int nb = min(CB, nc - c0);
        __syncthreads();
        // the first OB o values go out with the m, l loads
        float ov[OB];
#pragma unroll
        for (int j = 0; j < OB; ++j) ov[j] = j < nb ? read_f(ph + size_t(c0 + j) * pstride + 2 + d) : 0.0f;
        for (int i = tid; i < HPB * nb; i += kBlock) {
            const int h2 = min(blockIdx.x * HPB + i / nb, heads - 1);
            const float* pp = part + (size_t(h2) * a.max_chunks + c0 + i % nb) * pstride;
            m_s[i / nb][i % nb] = read_f(pp);
            l_s[i / nb][i % nb] = read_f(pp + 1);
        }
        __syncthreads();
        if (nc <= CB)
            for (int c = 0; c < nb; ++c) M = fmaxf(M, m_s[hl][c]);
        __syncthreads();
        // a_c in place of m_c: thread d of head hl takes chunks d, d + D, ...
        for (int c = d; c < nb; c += D) m_s[hl][c] = spec_expf(m_s[hl][c] - M);
        __syncthreads();
        for (int cb = 0; cb < nb; cb += OB) {
            if (cb > 0) {
#pragma unroll
                for (int j = 0; j < OB; ++j)
                    ov[j] = cb + j < nb ? read_f(ph + size_t(c0 + cb + j) * pstride + 2 + d) : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < OB; ++j)
                if (cb + j < nb) {
                    const float al = m_s[hl][cb + j];
                    L = __builtin_fmaf(al, l_s[hl][cb + j], L);
                    O = __builtin_fmaf(al, ov[j], O);
                }
        }
    }
    if (live) a.out[size_t(z) * size_t(heads) * D + size_t(hh) * D + d] = O * (1.0f / L);
}

// The batched step's attention epilogue: block z forms sequence z's output
// row -- the chunk combine of attention_combine_kernel for every (head, dim),
// same arithmetic, or the row attention_kernel combined in-block when one
// block held the whole context -- and quantizes it as the row kernels do (the row's
// maximum |value|, floored at 1e-5; quant_i8 with 127 / amax; columns
// de-interleaved per 8), so the o projection reads it as its GEMM input.
// Thread t holds (head t / D + HPP * i, dim t % D) for i < NO.
constexpr int kCombineThreads = 1024;
constexpr int kCombineMaxHeads = 64;
constexpr int kCombineBatch = 64;      // chunks whose a_c, l_c are staged at once
template <int D>
__global__ __launch_bounds__(kCombineThreads) void batch_combine_quant_kernel(AttnParams a)
{
    constexpr int C = kAttnChunk;
    constexpr int T = kCombineThreads;
    constexpr int HPP = T / D;                         // heads per pass
    constexpr int NO = kCombineMaxHeads / HPP;         // outputs per thread
    constexpr int CB = kCombineBatch;
    constexpr int pstride = D + 2;
    __shared__ float mx_s[NO][T / kWave];
    __shared__ float M_s[kCombineMaxHeads];
    __shared__ float al_s[kCombineMaxHeads][CB];
    __shared__ float l_s[kCombineMaxHeads][CB];
    __shared__ float wred[T / kWave];
    const int z = blockIdx.x;
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid & (kWave - 1);
    const int d = tid % D, h0 = tid / D;
    const int H = a.kv_heads * a.groups;
    const int cap = a.table->capacity[z];
    const int n = min(max(*a.table->position[z], 0), cap - 1) + 1;
    const int nc = (n + C - 1) / C;
    float val[NO];
    if (nc <= a.cpb) {
        // one block held every chunk of each head and combined them itself
        const float* row = a.out + size_t(z) * H * D;
#pragma unroll
        for (int i = 0; i < NO; ++i) {
            const int hh = h0 + HPP * i;
            val[i] = hh < H ? row[hh * D + d] : 0.0f;
        }
    } else {
        const float* part = a.part + size_t(z) * H * size_t(a.max_chunks) * pstride;
        static_assert(D % kWave == 0, "a head's threads are whole waves");
        if (nc > CB) {
            // M over every chunk first (several staged batches follow):
            // thread d of a head takes chunks d, d + D, ...
            float mm[NO];
#pragma unroll
            for (int i = 0; i < NO; ++i) mm[i] = -__builtin_inff();
            for (int c = d; c < nc; c += D)
#pragma unroll
                for (int i = 0; i < NO; ++i)
                    mm[i] = fmaxf(mm[i], part[(size_t(min(h0 + HPP * i, H - 1)) * a.max_chunks + c) * pstride]);
#pragma unroll
            for (int i = 0; i < NO; ++i) {
                mm[i] = wave_max64_all(mm[i]);
                if (lane == 0) mx_s[i][wave] = mm[i];
            }
            lds_sync();
            if (d == 0) {
#pragma unroll
                for (int i = 0; i < NO; ++i) {
                    const int hh = h0 + HPP * i;
                    if (hh >= H) continue;
                    float m2 = mx_s[i][h0 * (D / kWave)];
                    for (int w = 1; w < D / kWave; ++w) m2 = fmaxf(m2, mx_s[i][h0 * (D / kWave) + w]);
                    M_s[hh] = m2;
                }
            }
        }
        float L[NO], O[NO];
#pragma unroll
        for (int i = 0; i < NO; ++i) L[i] = O[i] = 0.0f;
        for (int c0 = 0; c0 < nc; c0 += CB) {
            const int nb = min(CB, nc - c0);
            // the o values of the batch's first 8 chunks go out with its m, l
            float ov[NO][8];
#pragma unroll
            for (int i = 0; i < NO; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    ov[i][j] = (h0 + HPP * i < H && j < nb)
                                   ? part[(size_t(h0 + HPP * i) * a.max_chunks + c0 + j) * pstride + 2 + d]
                                   : 0.0f;
            lds_sync();   // M_s written / the previous batch's staged values read
            for (int idx = tid; idx < H * nb; idx += T) {
                const int hh = idx / nb, c = idx - hh * nb;
                const float* pp = part + (size_t(hh) * a.max_chunks + c0 + c) * pstride;
                al_s[hh][c] = pp[0];
                l_s[hh][c] = pp[1];
            }
            lds_sync();
            if (nc <= CB) {
                for (int hh = tid; hh < H; hh += T) {
                    float m2 = al_s[hh][0];
                    for (int c = 1; c < nb; ++c) m2 = fmaxf(m2, al_s[hh][c]);
                    M_s[hh] = m2;
                }
                lds_sync();
            }
            // a_c = exp(m_c - M) in place of m_c
            for (int idx = tid; idx < H * nb; idx += T) {
                const int hh = idx / nb, c = idx - hh * nb;
                al_s[hh][c] = spec_expf(al_s[hh][c] - M_s[hh]);
            }
            lds_sync();
            for (int c = 0; c < nb; c += 8) {
                if (c > 0) {
#pragma unroll
                    for (int i = 0; i < NO; ++i)
#pragma unroll
                        for (int j = 0; j < 8; ++j)
                            ov[i][j] = (h0 + HPP * i < H && c + j < nb)
                                           ? part[(size_t(h0 + HPP * i) * a.max_chunks + c0 + c + j) * pstride + 2 + d]
                                           : 0.0f;
                }
#pragma unroll
                for (int i = 0; i < NO; ++i) {
                    const int hh = h0 + HPP * i;
                    if (hh >= H) continue;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        if (c + j < nb) {
                            const float al = al_s[hh][c + j];
                            L[i] = __builtin_fmaf(al, l_s[hh][c + j], L[i]);
                            O[i] = __builtin_fmaf(al, ov[i][j], O[i]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < NO; ++i) val[i] = h0 + HPP * i < H ? O[i] * (1.0f / L[i]) : 0.0f;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NO; ++i) amax = fmaxf(amax, fabsf(val[i]));   // 0 past the heads
    amax = wave_max64_all(amax);
    if (lane == 0) wred[wave] = amax;
    lds_sync();
    amax = wred[0];
#pragma unroll
    for (int w = 1; w < T / kWave; ++w) amax = fmaxf(amax, wred[w]);
    amax = fmaxf(amax, 1e-5f);
    const float inv = 127.0f / amax;
#pragma unroll
    for (int i = 0; i < NO; ++i) {
        const int hh = h0 + HPP * i;
        if (hh < H) a.q8[bq_pos(z, xq_offset(hh * D + d), a.kp)] = quant_i8(val[i], inv);
    }
    if (tid == 0) a.act[z] = amax / 127.0f;
}

size_t attention_workspace_floats(int heads, int max_chunks, int head_dim)
{
    return size_t(heads) * size_t(max_chunks) * size_t(head_dim + 2);
}

// One chunk per block: the most blocks in flight (1024 positions: 13.6 us
// against 25.5 us with four chunks per block, 4096: 25.9 against 33.2).
constexpr int kChunksPerBlock = 1;

int attention_splits(int context)
{
    const int nc = (context + kAttnChunk - 1) / kAttnChunk;
    return (nc + kChunksPerBlock - 1) / kChunksPerBlock;
}

template <int D, int GMAX, bool STEP>
static hipError_t launch_attn(const AttnParams& a, hipStream_t s)
{
    const int batch = (!STEP && a.batch > 1) ? a.batch : 1;
    const int splits = (a.max_chunks + kChunksPerBlock - 1) / kChunksPerBlock;
    hipLaunchKernelGGL((attention_kernel<D, GMAX, STEP, kChunksPerBlock>), dim3(a.kv_heads, splits, batch),
                       dim3(kBlock), 0, s, a);
    if (a.max_chunks > 1) {
        constexpr int hpb = kBlock / D;
        const int heads = a.kv_heads * a.groups;
        hipLaunchKernelGGL((attention_combine_kernel<D, STEP>), dim3((heads + hpb - 1) / hpb, batch), dim3(kBlock),
                           0, s, a);
    }
    return hipGetLastError();
}

hipError_t launch_batch_attention(const AttnParams& a, hipStream_t s)
{
    if (a.head_dim != 128 || !a.table || !a.qkv || !a.q8 || !a.act || a.groups > 8 ||
        a.kv_heads * a.groups > kCombineMaxHeads || a.batch < 1)
        return hipErrorInvalidValue;
    // one chunk per block while the grid fits about one round of the chip
    // (four 256-thread blocks per CU), else two; at most kAttnMaxSplits
    // splits in the grid (blocks walk the further ones)
    if (a.batch >= kSeqMinBatch && a.kv_heads == kAttnTailParts && a.groups == 4 && a.max_chunks <= kSeqChunks &&
        a.ll_max && a.epoch_ctr && a.epoch_id >= 0 && a.epoch_id < 256) {
        // one block per (sequence, kv head), the combine and quantization in it
        hipLaunchKernelGGL(seq_attention_kernel, dim3(a.batch * a.kv_heads), dim3(kSeqThreads), 0, s, a);
        return hipGetLastError();
    }
    AttnParams b = a;
    b.cpb = a.kv_heads * min(a.max_chunks, kAttnMaxSplits) * a.batch <= 1024 ? 1 : 2;
    const dim3 grid(a.kv_heads, min((a.max_chunks + b.cpb - 1) / b.cpb, kAttnMaxSplits), a.batch);
    const int H = a.kv_heads * a.groups;
    if (a.ll_part && a.ll_out && a.ll_max && a.epoch_ctr && a.epoch_id >= 0 && a.epoch_id < 256 &&
        a.groups <= 4 && H % (2 * kAttnTailParts) == 0 &&
        H <= 2 * kAttnTailNO * kAttnTailParts && int(grid.x * grid.y * grid.z) >= kAttnTailParts * a.batch) {
        // the combine and quantization in the launch's last blocks (BIG:
        // contexts of more than kAttnTailChunks chunks, split walk)
        if (a.max_chunks > kAttnTailChunks) {
            if (b.cpb == 1) hipLaunchKernelGGL((attention_kernel<128, 4, false, 1, true, true>), grid, dim3(kBlock), 0, s, b);
            else hipLaunchKernelGGL((attention_kernel<128, 4, false, 2, true, true>), grid, dim3(kBlock), 0, s, b);
        } else {
            if (b.cpb == 1) hipLaunchKernelGGL((attention_kernel<128, 4, false, 1, true>), grid, dim3(kBlock), 0, s, b);
            else hipLaunchKernelGGL((attention_kernel<128, 4, false, 2, true>), grid, dim3(kBlock), 0, s, b);
        }
        return hipGetLastError();
    }
    if ((a.max_chunks + b.cpb - 1) / b.cpb > kAttnMaxSplits) {   // the split walk
        if (b.cpb == 1) {
            if (a.groups <= 4) hipLaunchKernelGGL((attention_kernel<128, 4, false, 1, false, true>), grid, dim3(kBlock), 0, s, b);
            else hipLaunchKernelGGL((attention_kernel<128, 8, false, 1, false, true>), grid, dim3(kBlock), 0, s, b);
        } else {
            if (a.groups <= 4) hipLaunchKernelGGL((attention_kernel<128, 4, false, 2, false, true>), grid, dim3(kBlock), 0, s, b);
            else hipLaunchKernelGGL((attention_kernel<128, 8, false, 2, false, true>), grid, dim3(kBlock), 0, s, b);
        }
    } else if (b.cpb == 1) {
        if (a.groups <= 4) hipLaunchKernelGGL((attention_kernel<128, 4, false, 1>), grid, dim3(kBlock), 0, s, b);
        else hipLaunchKernelGGL((attention_kernel<128, 8, false, 1>), grid, dim3(kBlock), 0, s, b);
    } else {
        if (a.groups <= 4) hipLaunchKernelGGL((attention_kernel<128, 4, false, 2>), grid, dim3(kBlock), 0, s, b);
        else hipLaunchKernelGGL((attention_kernel<128, 8, false, 2>), grid, dim3(kBlock), 0, s, b);
    }
    hipLaunchKernelGGL(batch_combine_quant_kernel<128>, dim3(a.batch), dim3(kCombineThreads), 0, s, b);
    return hipGetLastError();
}

hipError_t launch_batch_qkv_attention(const int8_t* x, const float* act, const uint8_t* w, const float* ws, int k,
                                      const AttnParams& a, hipStream_t s)
{
    const int H = a.kv_heads * a.groups;
    const int rows = (H + 2 * a.kv_heads) * a.head_dim;
    if (a.batch >= kSeqMinBatch) return hipErrorNotSupported;   // (seq_attention_kernel's batches)
    if (!a.qkv_ll || !a.ll_part || !a.ll_out || !a.ll_max || !a.epoch_ctr || a.epoch_id < 0 || a.epoch_id >= 256 ||
        a.head_dim != 128 || !a.table || !a.qkv || !a.q8 || !a.act || a.batch < 1 || a.batch > 16 ||
        a.groups > 4 || H % (2 * kAttnTailParts) != 0 ||
        H > 2 * kAttnTailNO * kAttnTailParts || (k >> 1) > 1280 || (k & 31))
        return hipErrorNotSupported;
    AttnParams b = a;
    b.cpb = a.kv_heads * min(a.max_chunks, kAttnMaxSplits) * a.batch <= 1024 ? 1 : 2;
    const int gy = min((a.max_chunks + b.cpb - 1) / b.cpb, kAttnMaxSplits);
    if (a.kv_heads * gy * a.batch < kAttnTailParts * a.batch) return hipErrorNotSupported;
    GemmParams p{};
    p.m = a.batch;
    p.x = x;
    p.act = act;
    p.w = w; p.ws = ws;
    p.n = rows; p.k = k; p.kp = gemm_padded_k(k);
    p.tail.ll = a.qkv_ll;
    p.tail.epoch_ctr = a.epoch_ctr;
    p.tail.epoch_id = a.epoch_id;
    // one 16-wide sequence tile, 16 rows per block (at M = 32 the launch's
    // 960 blocks did not all fit on the chip at once: 3.08 -> 3.24 ms per
    // step, where M = 8 gained 2.04 -> 1.93 ms)
    const int tiles = (rows + 15) / 16;
    const dim3 grid(tiles + a.kv_heads * gy * a.batch);
    if (a.max_chunks > kAttnTailChunks) {   // the split walk and the batched tail combine
        if (b.cpb == 1) hipLaunchKernelGGL((qkv_attention_kernel<1, 1, 1, true>), grid, dim3(kBlock), 0, s, p, b, tiles, gy);
        else hipLaunchKernelGGL((qkv_attention_kernel<1, 1, 2, true>), grid, dim3(kBlock), 0, s, p, b, tiles, gy);
    } else {
        if (b.cpb == 1) hipLaunchKernelGGL((qkv_attention_kernel<1, 1, 1, false>), grid, dim3(kBlock), 0, s, p, b, tiles, gy);
        else hipLaunchKernelGGL((qkv_attention_kernel<1, 1, 2, false>), grid, dim3(kBlock), 0, s, p, b, tiles, gy);
    }
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
    case 128:
        // up to four query heads per kv head (Qwen3-4B's 32/8): the V
        // accumulation then runs two (head, dim) pairs per thread, not four
        return a.groups <= 4 ? launch_attn<128, 4, false>(a, s) : launch_attn<128, 8, false>(a, s);
    default: return hipErrorInvalidValue;
    }
}

// ---- the drop-in GQA decode in one launch ------------------------------------------
//
// hq_gqa_decode's kernel: block i < nc * kv is chunk item (chunk c = i / kv,
// kv head g = i % kv); the launch's last blocks combine.  An item block
// copies its chunk's K and V rows (64 rows of 2D bytes each) straight into
// LDS with global->LDS loads (no register round trip), loads its kv head's
// G query heads into registers meanwhile, and computes, in the spec order
// of or_gqa_decode_split: the scores (16 partial fmaf chains of D/16 dims,
// the 16-lane halving tree, times 1 / sqrt(D)), the chunk's max m, e_t =
// exp(s_t - m) and l = the 64-slot tree, and o[d] = the fmaf chain of e_t *
// v_t[d] over ascending t.  A one-chunk context finishes there (out = o *
// (1 / l) through the combine's operations); otherwise the item publishes
// (m, l, o[0..D-1]) per query head as 32-bit words holding the value's bits
// XOR kGqaKey (a signalling-NaN pattern no arithmetic result carries, so a
// published word is never 0) with agent-scope stores.  A combine block
// (256 / D query heads, one thread per (head, dim) chain) waits for those
// words -- one lane per head first watches the last chunk's last word (the
// last items start last), then every thread polls its own words -- and runs
// the spec's combine over ascending chunks: M = max m_c, a_c = exp(m_c - M),
// L = fmaf(a_c, l_c, L), O = fmaf(a_c, o_c[d], O), out = O * (1 / L); it
// then stores 0 over every word it read.  The words therefore start and end
// every call at zero: the workspace must be zero-filled before its first
// use, and calls that share a workspace must not overlap.  Every wait is
// bounded (kGqaSpinLimit rounds), so the launch always ends.
constexpr uint32_t kGqaKey = 0x7FA5A5A5u;
constexpr unsigned kGqaSpinLimit = 1u << 22;

__device__ __forceinline__ void gqa_word_store(uint32_t* p, float v)
{
    __hip_atomic_store(p, f32_bits(v) ^ kGqaKey, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t gqa_word_load(const uint32_t* p)
{
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void gqa_word_clear(uint32_t* p)
{
    __hip_atomic_store(p, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The value of word *p once it is published (bounded wait).
__device__ __forceinline__ float gqa_word_wait(const uint32_t* p, unsigned& budget)
{
    uint32_t w = gqa_word_load(p);
    while (w == 0u && budget != 0u) {
        __builtin_amdgcn_s_sleep(1);
        if (--budget == 0u) break;
        w = gqa_word_load(p);
    }
    return bits_f32(w ^ kGqaKey);
}

constexpr int kFlashThreads = 512;   // threads of a gqa_flash_kernel block (8 waves)

template <int D, int GMAX>
struct FlashLds {
    alignas(16) uint16_t k[kAttnChunk * D];   // the chunk's K rows [t][d]
    alignas(16) uint16_t v[kAttnChunk * D];   // and V rows
    alignas(16) float e[GMAX][kAttnChunk];    // scores, then exp terms
    alignas(16) float q[GMAX * D];            // the kv head's query rows
    float m[GMAX], l[GMAX];
};

struct FlashParams {
    const float* q;           // [kv * G, D]
    const uint16_t* keys;     // [context, kv, D] fp16
    const uint16_t* values;
    uint32_t* words;          // published partials (zero between calls), nc4 = nc rounded up to 4,
                              // U = combine units per head: o [kv * G][nc4 / 4][D][4], then
                              // m [kv * G][U][nc4], then l [kv * G][U][nc4] (one copy per unit)
    float* out;               // [kv * G, D]
    long long time_stride;    // elements per position (kv * D)
    int n, nc, kv, G;
};

// DPL consecutive halves of an LDS row as fp32.
template <int DPL>
__device__ __forceinline__ void lds_halves(const uint16_t* p, float (&k)[DPL])
{
    if constexpr (DPL == 8) {
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) { k[2 * j] = f16_to_f32(uint16_t(w[j])); k[2 * j + 1] = f16_to_f32(uint16_t(w[j] >> 16)); }
    } else if constexpr (DPL == 4) {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        k[0] = f16_to_f32(uint16_t(v.x)); k[1] = f16_to_f32(uint16_t(v.x >> 16));
        k[2] = f16_to_f32(uint16_t(v.y)); k[3] = f16_to_f32(uint16_t(v.y >> 16));
    } else if constexpr (DPL == 2) {
        const uint32_t v = *reinterpret_cast<const uint32_t*>(p);
        k[0] = f16_to_f32(uint16_t(v)); k[1] = f16_to_f32(uint16_t(v >> 16));
    } else {
        k[0] = f16_to_f32(*p);
    }
}

template <int D>
constexpr int flash_units_per_head() { return D == 128 ? 2 : 1; }

template <int D, int GMAX>
__device__ void flash_item(const FlashParams& a, FlashLds<D, GMAX>& S, int c, int g)
{
    constexpr int C = kAttnChunk;
    constexpr int T = kFlashThreads;
    constexpr int NW = T / kWave;                        // waves
    constexpr int DPL = D / 16;                          // dims per score lane
    constexpr int HSTEP = T / D;                         // heads between a thread's V chains
    constexpr int PAIRS = (GMAX * D + T - 1) / T;
    constexpr int REPS = C / (T / 16);                   // score positions per 16-lane group
    constexpr int RPI = 1024 / (2 * D);                  // K rows per 1 KB copy instruction
    constexpr int LPR = 2 * D / 16;                      // lanes per row in a copy
    constexpr int NINS = C / RPI;                        // copy instructions per matrix
    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid & (kWave - 1);
    const int G = a.G;
    const int t0 = c * C;
    const int tn = min(C, a.n - t0);
    // The kv head's G query rows, then K rows, then V rows, straight into
    // LDS, all by global->LDS copies (a wave's loads complete in issue
    // order, and the compiler tracks none of these, so its own waits do not
    // hold the scores back for V).  K/V instruction `ins` moves rows RPI*ins
    // .. +RPI-1, lane i row RPI*ins + i/LPR, bytes 16(i%LPR)..; rows past the
    // context re-read the last one (never used).  The scores run once K is
    // in, while V is still arriving.
    {
        const int qbytes = G * D * 4;
        const float* qb = a.q + size_t(g) * G * D;
        for (int ins = wave; ins * 1024 < qbytes; ins += NW)
            dma16(qb, uint32_t(min(ins * 1024 + lane * 16, qbytes - 16)), lds_addr(S.q) + uint32_t(ins) * 1024u);
    }
    const int nq = wave * 1024 < G * D * 4 ? 1 : 0;   // this wave's q copies (G * D * 4 <= 4 KB < NW KB)
    const uint16_t* kb = a.keys + size_t(t0) * size_t(a.time_stride) + size_t(g) * D;
    const uint16_t* vb = a.values + size_t(t0) * size_t(a.time_stride) + size_t(g) * D;
    auto copy_off = [&](int ins) {
        const int row = min(RPI * ins + lane / LPR, tn - 1);
        return uint32_t(size_t(row) * size_t(a.time_stride) * 2u) + uint32_t(lane % LPR) * 16u;
    };
    for (int ins = wave; ins < NINS; ins += NW) dma16(kb, copy_off(ins), lds_addr(S.k) + uint32_t(ins) * 1024u);
    for (int ins = wave; ins < NINS; ins += NW) dma16(vb, copy_off(ins), lds_addr(S.v) + uint32_t(ins) * 1024u);
    // this wave's q and K copies are done when at most its V copies are
    // outstanding (memory operations complete in issue order)
    constexpr int VMAX = (NINS + NW - 1) / NW;
    static_assert(VMAX <= 2, "wait_vm_le covers up to two outstanding copies");
    static_assert(GMAX * D * 4 <= NW * 1024, "one q copy per wave at most");
    (void)nq;
    wait_vm_le(wave < NINS ? (NINS - 1 - wave) / NW + 1 : 0);
    lds_sync();
    // this lane's DPL dims of every query head (a head past G repeats G - 1)
    const int l16 = tid & 15, grp = tid >> 4;
    float qr[GMAX][DPL];
#pragma unroll
    for (int h = 0; h < GMAX; ++h)
#pragma unroll
        for (int j = 0; j < DPL; ++j) qr[h][j] = S.q[min(h, G - 1) * D + l16 * DPL + j];
    // scores, 16 lanes per position.  Every lane computes every head and
    // row (a head past G repeats head G - 1, a row past the context repeats
    // the last one; neither is stored), so no branch splits the REPS x GMAX
    // independent fmaf chains and trees; lane 0 of each row stores.
    const float scale = 1.0f / __builtin_sqrtf(float(D));
    float dot[REPS][GMAX];
#pragma unroll
    for (int rep = 0; rep < REPS; ++rep) {
        float k[DPL];
        lds_halves<DPL>(S.k + (grp + (T / 16) * rep) * D + l16 * DPL, k);
#pragma unroll
        for (int h = 0; h < GMAX; ++h) {
            float pp = 0.0f;
#pragma unroll
            for (int j = 0; j < DPL; ++j) pp = __builtin_fmaf(qr[h][j], k[j], pp);
            dot[rep][h] = pp;
        }
    }
#pragma unroll
    for (int rep = 0; rep < REPS; ++rep)
#pragma unroll
        for (int h = 0; h < GMAX; ++h) dot[rep][h] = row_tree_sum16(dot[rep][h]);
    if (l16 == 0) {
#pragma unroll
        for (int rep = 0; rep < REPS; ++rep) {
            const int i = grp + (T / 16) * rep;
#pragma unroll
            for (int h = 0; h < GMAX; ++h) S.e[h][i] = i < tn ? dot[rep][h] * scale : -__builtin_inff();
        }
    }
    lds_sync();
    // chunk statistics, one wave per head
    for (int h = wave; h < G; h += NW) {
        const float sc = S.e[h][lane];
        const float m = wave_max64_all(sc);
        const float e = lane < tn ? spec_expf(sc - m) : 0.0f;
        const float l = wave_tree_sum64(e);
        S.e[h][lane] = e;
        if (lane == 0) { S.m[h] = m; S.l[h] = l; }
    }
    wait_all_memory();   // this wave's V copies have landed
    lds_sync();
    // V: thread (h0, d) runs the chains of heads h0, h0 + HSTEP, ...; the
    // exp terms are read four positions at a time
    const int d = tid % D, h0 = tid / D;
    float o[PAIRS];
#pragma unroll
    for (int r = 0; r < PAIRS; ++r) o[r] = 0.0f;
    int i = 0;
    for (; i + 8 <= tn; i += 8) {
        float v[8];
        float4 e[PAIRS][2];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = f16_to_f32(S.v[(i + j) * D + d]);
#pragma unroll
        for (int r = 0; r < PAIRS; ++r) {
            const float* er = &S.e[min(h0 + HSTEP * r, GMAX - 1)][i];
            e[r][0] = *reinterpret_cast<const float4*>(er);
            e[r][1] = *reinterpret_cast<const float4*>(er + 4);
        }
#pragma unroll
        for (int r = 0; r < PAIRS; ++r) {
            o[r] = __builtin_fmaf(e[r][0].x, v[0], o[r]);
            o[r] = __builtin_fmaf(e[r][0].y, v[1], o[r]);
            o[r] = __builtin_fmaf(e[r][0].z, v[2], o[r]);
            o[r] = __builtin_fmaf(e[r][0].w, v[3], o[r]);
            o[r] = __builtin_fmaf(e[r][1].x, v[4], o[r]);
            o[r] = __builtin_fmaf(e[r][1].y, v[5], o[r]);
            o[r] = __builtin_fmaf(e[r][1].z, v[6], o[r]);
            o[r] = __builtin_fmaf(e[r][1].w, v[7], o[r]);
        }
    }
    for (; i < tn; ++i) {
        const float v = f16_to_f32(S.v[i * D + d]);
#pragma unroll
        for (int r = 0; r < PAIRS; ++r) o[r] = __builtin_fmaf(S.e[min(h0 + HSTEP * r, GMAX - 1)][i], v, o[r]);
    }
#pragma unroll
    for (int r = 0; r < PAIRS; ++r) {
        const int h = h0 + HSTEP * r;
        if (h >= G) continue;
        const int qh = g * G + h;
        if (a.nc == 1) {
            // the combine's operations over the one chunk
            const float al = spec_expf(S.m[h] - S.m[h]);
            const float L = __builtin_fmaf(al, S.l[h], 0.0f);
            const float O = __builtin_fmaf(al, o[r], 0.0f);
            a.out[size_t(qh) * D + d] = O * (1.0f / L);
        } else {
            const size_t nc4 = size_t((a.nc + 3) & ~3), H = size_t(a.kv) * G;
            uint32_t* ow = a.words + (size_t(qh) * nc4 + (c & ~3)) * D + size_t(d) * 4;
            gqa_word_store(ow + (c & 3), o[r]);
            // the last chunk also publishes 0.0 into its group's padding slots
            if (c == a.nc - 1)
                for (int p = (c & 3) + 1; p < 4; ++p) gqa_word_store(ow + p, 0.0f);
            // m and l once per combine unit of the head: each unit clears
            // the copy it reads
            constexpr int U = flash_units_per_head<D>();
            if (d < U) {
                gqa_word_store(a.words + H * nc4 * D + (size_t(qh) * U + d) * nc4 + c, S.m[h]);
                gqa_word_store(a.words + H * nc4 * (D + U) + (size_t(qh) * U + d) * nc4 + c, S.l[h]);
            }
        }
    }
}

// Combine blocks: wave 0 of each runs one unit -- (query head, half of its
// dims) for D = 128, a query head for D <= 64 (lanes past D run the chunk
// roles only); the other waves leave at once, so the units' loads and
// clears issue from as many CUs as there are units.  Per batch of 64
// chunks, lane c holds chunk c's m_c and l_c, so M is one wave max and a_c
// = exp(m_c - M) is computed in lane c; the chain reads a_c and l_c from
// lane c (readlane), with no LDS and no barrier.  A batch's words are
// fetched in one burst (the lane's o_c[d] and its m_c, l_c), the
// unpublished ones polled again, and cleared once held.  Chunks past the
// context enter the chain as a_c = 0, l_c = 0, o_c = 0: fmaf(0, 0, x)
// returns x, and neither L nor O is ever -0 (their terms' zeros are +0
// sums), so the padding leaves the bits unchanged.  With more than one
// batch M comes from a first pass over every m_c.
constexpr int kFlashCB = 64;   // chunks per batch: one per lane


template <int D>
__device__ void flash_combine(const FlashParams& a, int unit)
{
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    constexpr int NG = kFlashCB / 4;          // chunk groups per batch
    const int lane = threadIdx.x & (kWave - 1);
    const int hraw = unit / flash_units_per_head<D>();
    const int half = unit % flash_units_per_head<D>();
    const int d = half * kWave + lane;        // this lane's dim (a chain when d < D)
    const bool chain = d < D;
    const int nc = a.nc;
    const size_t nc4 = size_t((nc + 3) & ~3), H = size_t(a.kv) * a.G;
    uint32_t* obase = a.words + size_t(hraw) * nc4 * D;              // [nc4 / 4][D][4]
    constexpr int U = flash_units_per_head<D>();
    uint32_t* mbase = a.words + H * nc4 * D + size_t(unit) * nc4;    // this unit's copy [nc4]
    uint32_t* lbase = a.words + H * nc4 * (D + U) + size_t(unit) * nc4;
    unsigned budget = kGqaSpinLimit;
    float M = -__builtin_inff();
    if (nc > kFlashCB) {
        float mm = -__builtin_inff();
        for (int c = lane; c < nc; c += kWave) mm = fmaxf(mm, gqa_word_wait(mbase + c, budget));
        M = wave_max64_all(mm);
    }
    float L = 0.0f, O = 0.0f;
    for (int c0 = 0; c0 < nc; c0 += kFlashCB) {
        const int nb = min(kFlashCB, nc - c0);
        const int ngrp = (nb + 3) >> 2;          // chunk groups of the batch
        // every load unconditional, through buffer descriptors that end at
        // the batch's last chunk (group): a load past one returns 0 without
        // touching memory and a store there is dropped.  Group g4's four
        // chunks of dim d are one 16-byte word of the lane, at a constant
        // scalar offset; a group's padding slots past the context hold a
        // published 0.0 (written by the last chunk's item), groups past the
        // batch are set to 0.0 here, and lanes past D (D < 64) read dim 0's
        // words and discard them.
        const __amdgpu_buffer_rsrc_t ro = raw_rsrc(obase + size_t(c0) * D, ngrp * D * 16);
        const __amdgpu_buffer_rsrc_t rm = raw_rsrc(mbase + c0, nb * 4);
        const __amdgpu_buffer_rsrc_t rl = raw_rsrc(lbase + c0, nb * 4);
        const uint32_t vo = uint32_t(chain ? d : 0) * 16u;
        // first the batch's m_c and l_c, one chunk per lane (two loads per
        // round): an item publishes them with its o words, so once every
        // chunk's are in, the o burst below rarely meets an empty word
        const bool mine = lane < nb;             // lane c's chunk
        uint32_t mw = 0u, lw = 0u;
        while (true) {
            mw = mw != 0u ? mw : __builtin_amdgcn_raw_buffer_load_b32(rm, lane * 4, 0, kAgentSC1);
            lw = lw != 0u ? lw : __builtin_amdgcn_raw_buffer_load_b32(rl, lane * 4, 0, kAgentSC1);
            mw = mine ? mw : f32_bits(-__builtin_inff()) ^ kGqaKey;
            lw = mine ? lw : kGqaKey;
            if (!__builtin_amdgcn_ballot_w64((mw == 0u) | (lw == 0u)) || budget == 0u) break;   // (wave-uniform)
            __builtin_amdgcn_s_sleep(1);
            --budget;
        }
        v4u ow[NG];
#pragma unroll
        for (int g4 = 0; g4 < NG; ++g4) ow[g4] = __builtin_amdgcn_raw_buffer_load_b128(ro, vo, g4 * D * 16, kAgentSC1);
#pragma unroll
        for (int g4 = 0; g4 < NG; ++g4)
            if (g4 >= ngrp) ow[g4] = v4u{kGqaKey, kGqaKey, kGqaKey, kGqaKey};   // (wave-uniform)
        // poll what was not published yet (a published word keeps its value
        // for the rest of the call, so the whole burst is simply re-read;
        // the padding entries set above are nonzero and stay so)
        while (budget != 0u) {
            bool pending = false;
#pragma unroll
            for (int g4 = 0; g4 < NG; ++g4)
                pending |= (ow[g4][0] == 0u) | (ow[g4][1] == 0u) | (ow[g4][2] == 0u) | (ow[g4][3] == 0u);
            if (!pending) break;
            __builtin_amdgcn_s_sleep(1);
            --budget;
#pragma unroll
            for (int g4 = 0; g4 < NG; ++g4) {
                const v4u w = __builtin_amdgcn_raw_buffer_load_b128(ro, vo, g4 * D * 16, kAgentSC1);
#pragma unroll
                for (int j = 0; j < 4; ++j) ow[g4][j] = ow[g4][j] != 0u ? ow[g4][j] : w[j];
            }
        }
        const float mc = bits_f32(mw ^ kGqaKey);
        if (nc <= kFlashCB) M = wave_max64_all(mc);
        const float ac = mine ? spec_expf(mc - M) : 0.0f;
        const float lc = bits_f32(lw ^ kGqaKey);
#pragma unroll
        for (int c = 0; c < kFlashCB; ++c) {
            const float al = bits_f32(__builtin_amdgcn_readlane(f32_bits(ac), c));
            L = __builtin_fmaf(al, bits_f32(__builtin_amdgcn_readlane(f32_bits(lc), c)), L);
            O = __builtin_fmaf(al, bits_f32(ow[c >> 2][c & 3] ^ kGqaKey), O);
            // (the broadcasts stay next to their use: hoisted, 128 of them
            // would not fit the scalar registers)
            if ((c & 7) == 7) __builtin_amdgcn_sched_barrier(0);
        }
        // the words go back to 0 (each is read by this lane alone -- m_c and
        // l_c are this unit's own copies -- and the first pass over m_c
        // above is done)
        if (chain) {
#pragma unroll
            for (int g4 = 0; g4 < NG; ++g4)
                __builtin_amdgcn_raw_buffer_store_b128(v4u{0u, 0u, 0u, 0u}, ro, vo, g4 * D * 16, kAgentSC1);
        }
        if (mine) {
            __builtin_amdgcn_raw_buffer_store_b32(0u, rm, lane * 4, 0, kAgentSC1);
            __builtin_amdgcn_raw_buffer_store_b32(0u, rl, lane * 4, 0, kAgentSC1);
        }
    }
    if (chain) a.out[size_t(hraw) * D + d] = O * (1.0f / L);
}

template <int D, int GMAX>
__global__ __launch_bounds__(kFlashThreads) void gqa_flash_kernel(FlashParams a)
{
    __shared__ FlashLds<D, GMAX> lds;
    const int items = a.nc * a.kv;
    const int b = blockIdx.x;
    if (b < items) flash_item<D, GMAX>(a, lds, b / a.kv, b % a.kv);   // (block-uniform)
    else if (threadIdx.x < kWave) flash_combine<D>(a, b - items);
}

template <int D, int GMAX>
static void launch_flash(const FlashParams& a, hipStream_t s)
{
    const int H = a.kv * a.G;
    const int blocks = a.nc * a.kv + (a.nc > 1 ? H * flash_units_per_head<D>() : 0);
    hipLaunchKernelGGL((gqa_flash_kernel<D, GMAX>), dim3(blocks), dim3(kFlashThreads), 0, s, a);
}

// head_dim 16/32/64/128, groups <= 8 (checked by the caller)
static hipError_t launch_gqa_flash(const float* query, const uint16_t* keys, const uint16_t* values, uint32_t* words,
                                   float* output, int context, int kv_heads, int groups, int head_dim, hipStream_t s)
{
    FlashParams a{};
    a.q = query;
    a.keys = keys;
    a.values = values;
    a.words = words;
    a.out = output;
    a.time_stride = (long long)kv_heads * head_dim;
    a.n = context;
    a.nc = (context + kAttnChunk - 1) / kAttnChunk;
    a.kv = kv_heads;
    a.G = groups;
    switch (head_dim) {
    case 16: launch_flash<16, 8>(a, s); break;
    case 32: launch_flash<32, 8>(a, s); break;
    case 64: launch_flash<64, 8>(a, s); break;
    default:
        if (groups <= 4) launch_flash<128, 4>(a, s);
        else launch_flash<128, 8>(a, s);
    }
    return hipGetLastError();
}

}  // namespace hq

using namespace hq;

extern "C" size_t hq_gqa_workspace_bytes(int score_stride, int kv_heads, int groups, int head_dim)
{
    if (score_stride <= 0 || kv_heads <= 0 || groups <= 0 || head_dim <= 0) return 0;
    const int nc = (score_stride + kAttnChunk - 1) / kAttnChunk;
    // a 256-byte header (reserved), then the chunk partials of whole groups
    // of four chunks (D + 2 words per query head and chunk, and up to two
    // more for the combine units' own copies of m and l): one workspace
    // serves every context up to score_stride
    return 256 + attention_workspace_floats(kv_heads * groups, (nc + 3) & ~3, head_dim + 2) * 4;
}

// Checks and launch shared by hq_gqa_decode and hq_gqa_decode_noalloc.
static int gqa_check(const float* query, const uint16_t* keys, const uint16_t* values, const float* output,
                     int context, int kv_heads, int groups, int head_dim, int score_stride)
{
    if (!query || !keys || !values || !output) return HQ_ERR_ARG;
    if (context <= 0 || kv_heads <= 0 || groups <= 0 || groups > 8) return HQ_ERR_ARG;
    if (score_stride < context) return HQ_ERR_ARG;
    if (head_dim != 16 && head_dim != 32 && head_dim != 64 && head_dim != 128) return HQ_ERR_ARG;
    if (kv_heads > 64) return HQ_ERR_ARG;
    if ((reinterpret_cast<uintptr_t>(keys) & 15u) != 0 || (reinterpret_cast<uintptr_t>(values) & 15u) != 0)
        return HQ_ERR_ALIGN;
    return HQ_OK;
}

static int gqa_launch(const float* query, const uint16_t* keys, const uint16_t* values, void* workspace,
                      float* output, int context, int kv_heads, int groups, int head_dim, hipStream_t stream)
{
    uint32_t* words = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + 256);
    const hipError_t e = launch_gqa_flash(query, keys, values, words, output, context, kv_heads, groups, head_dim,
                                          stream);
    return e == hipSuccess ? HQ_OK : HQ_ERR_LAUNCH;
}

// The reference's argument list (litespark_int4.cpp:160-171): the K/V time
// stride is kv_heads * head_dim (:172), and score_stride is the row stride of
// its `scores` scratch, i.e. the context capacity that scratch was sized for
// (cpu_lightspark.py:405 passes state.capacity).  Here the workspace takes
// the scratch's place and is sized by the same number.
extern "C" int hq_gqa_decode(const float* query, const uint16_t* keys, const uint16_t* values,
                             void* workspace, float* output, int context, int kv_heads,
                             int groups, int head_dim, int score_stride, void* stream)
{
    const int st = gqa_check(query, keys, values, output, context, kv_heads, groups, head_dim, score_stride);
    if (st != HQ_OK) return st;
    if (!workspace) return HQ_ERR_ARG;
    if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return HQ_ERR_ALIGN;
    return gqa_launch(query, keys, values, workspace, output, context, kv_heads, groups, head_dim,
                      static_cast<hipStream_t>(stream));
}

// ---- the variant that allocates nothing ----------------------------------------
//
// For callers that cannot allocate device memory (code under HIP graph
// capture, serving loops that forbid hipMalloc): hq_gqa_decode with its
// workspace in a file-scope device array instead of a caller buffer.  Each
// GPU holds its own copy of `scratch` until the process ends.  The array's
// name is only a host-side stand-in: its device address is taken with
// hipGetSymbolAddress once per device, with that device current, and that
// address is what the kernels receive.  Every call on a device shares the
// device's array, so calls that overlap on one GPU race.
constexpr size_t kNoAllocScratchBytes = size_t(4) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mutex;

// The device address of this device's `scratch` (nullptr on failure).
static void* scratch_address(int dev)
{
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) return nullptr;
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
}

extern "C" int hq_gqa_decode_noalloc(const float* query, const uint16_t* keys, const uint16_t* values,
                                     float* output, int context, int kv_heads, int groups, int head_dim,
                                     int score_stride, void* stream)
{
    const int st = gqa_check(query, keys, values, output, context, kv_heads, groups, head_dim, score_stride);
    if (st != HQ_OK) return st;
    // the bytes this call uses (its context's chunk partials), not the
    // score_stride sizing of the caller-workspace form
    if (hq_gqa_workspace_bytes(context, kv_heads, groups, head_dim) > kNoAllocScratchBytes) return HQ_ERR_ARG;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return HQ_ERR_DEVICE;
    void* ws = scratch_address(dev);
    if (ws == nullptr) return HQ_ERR_DEVICE;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    return gqa_launch(query, keys, values, ws, output, context, kv_heads, groups, head_dim, s);
}
