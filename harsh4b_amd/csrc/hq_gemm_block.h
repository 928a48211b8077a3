// hq_gemm_block.h - the device side of the batched decode GEMM (int4
// weights x M int8 activation rows on v_mfma_i32_16x16x64_i8): its
// parameters, the LDS-staged block (gemm_lds_block) and the batched step's
// launch tails.  Included by hq_gemm.hip (the GEMM kernels and their host
// code) and hq_attention.hip (the batched step's qkv GEMM in the attention
// launch).
#pragma once

#include "hq_device.h"
#include "hq_internal.h"

namespace hq {


typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// 16-byte load that streams past the caches (the weights are read once)
__device__ __forceinline__ uint4 load16_nt(const uint8_t* p)
{
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

constexpr int kSlice = 256;       // activation rows are padded to whole slices of 256 columns
constexpr int kMaxBatch = 32;     // sequences per launch (two 16-wide B tiles)

struct GemmParams {
    const int8_t* x;          // [m, kp] de-interleaved per 8 columns, zero past K
    const float* act;         // [m]
    const uint8_t* w;         // [N, K/2]
    const float* ws;          // [N]
    float* out;               // [m, N]
    int32_t* acc_out;         // nullable [m, N]
    int m, n, k, kp;          // kp: padded row stride of x (a multiple of kSlice)
    // SwiGLU launches (gemm_lds_kernel<2, ..., true>): w holds gate rows
    // [0, n) then up rows [n, 2n); out [m, n] receives SwiGLU(gate, up) and
    // pmax [blocks, m] each block's maximum |out| per sequence
    float* pmax;
    // Tail launches (gemm_lds_kernel<..., TAIL = true>, the batched step's o
    // and down GEMMs): the outputs go to ll [m, n] as {value, epoch} entries
    // (epoch = *epoch_ctr << 8 | epoch_id, unique per launch of a step), and
    // the last blocks finish the rows: the residual add into x, RMSNorm with
    // gamma and quantization into q / act (o, down: one block per row), or the
    // quantization of the SwiGLU row with its maximum from the blocks' entries
    // in pmax (gate_up: four blocks per row).
    GemmTail tail;
};

// De-interleave 8 int8 columns (a, b = the two little-endian dwords) into
// [even columns | odd columns].
__device__ __forceinline__ void deinterleave8(uint32_t a, uint32_t b, uint32_t& ev, uint32_t& od)
{
    ev = (a & 0xFFu) | ((a >> 8) & 0xFF00u) | ((b & 0xFFu) << 16) | ((b & 0xFF0000u) << 8);
    od = ((a >> 8) & 0xFFu) | ((a >> 16) & 0xFF00u) | ((b & 0xFF00u) << 8) | (b & 0xFF000000u);
}

// ---- batched-step tails ------------------------------------------------------------

__device__ __forceinline__ uint32_t tail_epoch(const GemmTail& t)
{
    return (*t.epoch_ctr << 8) | uint32_t(t.epoch_id);
}

// Row s of a tail launch, by threads 0-255 of one block (the others only
// take the barriers): once every tile block's entry of the row is current
// (the tile blocks come first in index order and blocks start in index
// order, so the blocks a tail waits for are running or done), the same
// operations as the row kernel's RESID_NORM mode: x + GEMM output into the
// residual, RMSNorm (256 strided fmaf partials, halving tree), the
// normalized row's maximum over the four waves in order, quantization into
// the de-interleaved row and act = amax / 127.
template <int NPT>
__device__ void gemm_tail_row(const GemmParams& p, int s, uint32_t ep, float* red, float* wmax)
{
    const GemmTail& T = p.tail;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int k = p.n;
    const bool on = tid < kBlock;
    float* xr = T.x + size_t(s) * k;
    float v[NPT], gam[NPT];
    if (on) {
        const uint64_t* src = T.ll + size_t(s) * k;
        uint64_t e[NPT];
#pragma unroll
        for (int j = 0; j < NPT; ++j) {
            const int i = tid + kBlock * j;
            v[j] = i < k ? xr[i] : 0.0f;
            gam[j] = i < k ? T.gamma[i] : 0.0f;
            e[j] = i < k ? tail_load(src + i) : uint64_t(ep) << 32;
        }
        unsigned spins = 0;
        while (true) {
            bool pending = false;
            unrolled<NPT>([&](auto j) { pending |= !tail_ready(e[j], ep); });
            if (!pending) break;
            if (++spins == kTailSpinLimit) {
                atomicOr(T.table->status[s], HQ_STEP_SYNC);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
            unrolled<NPT>([&](auto j) {
                if (!tail_ready(e[j], ep)) e[j] = tail_load(src + tid + kBlock * j);
            });
        }
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < NPT; ++j) {
            const int i = tid + kBlock * j;
            v[j] = i < k ? v[j] + bits_f32(uint32_t(e[j])) : 0.0f;
            if (i < k) {
                xr[i] = v[j];   // the new residual (this block alone reads and writes row s)
                ss = __builtin_fmaf(v[j], v[j], ss);
            }
        }
        red[tid] = ss;
    }
    __syncthreads();
    if (on) {
        const float r2 = (red[lane] + red[lane + 128]) + (red[lane + 64] + red[lane + 192]);
        const float total = wave_tree_sum64_all(r2);
        const float r = __builtin_sqrtf(total / float(k) + T.eps);
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < NPT; ++j) {
            const int i = tid + kBlock * j;
            v[j] = i < k ? (v[j] / r) * gam[j] : 0.0f;
            amax = fmaxf(amax, fabsf(v[j]));
        }
        amax = wave_max64_all(amax);
        if (lane == 0) wmax[tid / kWave] = amax;
    }
    __syncthreads();
    if (on) {
        float amax = wmax[0];
#pragma unroll
        for (int w = 1; w < kBlock / kWave; ++w) amax = fmaxf(amax, wmax[w]);
        amax = fmaxf(amax, 1e-5f);
        const float inv = 127.0f / amax;
#pragma unroll
        for (int j = 0; j < NPT; ++j) {
            const int i = tid + kBlock * j;
            if (i < k) T.q[bq_pos(s, xq_offset(i), T.kq)] = quant_i8(v[j], inv);
        }
        if (tid == 0) T.act[s] = amax / 127.0f;
    }
}
// tail rows of up to 2560 values (wider rows hold more registers than a
// 1024-thread down launch has: they take the row kernel instead)
constexpr int kTailNPT = 10;

// Blocks of a tail launch that compute tiles (the rest finish rows).
template <bool SWIGLU>
__device__ __forceinline__ int tail_tiles(const GemmParams& p)
{
    return int(gridDim.x) - (SWIGLU ? 4 : 1) * p.m;
}

// Quarter qt of SwiGLU row s (values [qt*Q, qt*Q + Q), Q = 2560), by threads
// 0-255 of one block: the row's maximum |value| over the launch's block
// entries (order-free), then the same quantization as batch_act_quant_kernel
// (amax floored at 1e-5, quant_i8 with 127 / amax, de-interleaved per 8,
// act = amax / 127, written by quarter 0).
constexpr int kSwigluTailQ = kBlock * 10;   // values per tail block: rows of up to 4 * 2560
constexpr int kSwigluTailB = 3;             // block maxima per thread: up to 768 blocks
__device__ inline void gemm_swiglu_tail_row(const GemmParams& p, int s, int qt, uint32_t ep, float* wmax)
{
    const GemmTail& T = p.tail;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int nb = tail_tiles<true>(p);   // the tile blocks' maxima
    const int n = p.n;
    const bool on = tid < kBlock;
    // this block's values, requested with the block maxima
    const int i0 = qt * kSwigluTailQ + tid;
    const uint64_t* vsrc = T.ll + size_t(s) * n;
    const uint64_t ready = uint64_t(ep) << 32;
    uint64_t e[10], mb[kSwigluTailB];
    float mx = 0.0f;
    if (on) {
        unrolled<10>([&](auto j) {
            const int i = i0 + kBlock * j;
            e[j] = i < n ? tail_load(vsrc + i) : ready;
        });
        unrolled<kSwigluTailB>([&](auto j) {
            const int b = tid + kBlock * j;
            mb[j] = b < nb ? tail_load(T.pmax + size_t(b) * p.m + s) : ready;
        });
        unsigned spins = 0;
        while (true) {
            bool pending = false;
            unrolled<kSwigluTailB>([&](auto j) { pending |= !tail_ready(mb[j], ep); });
            unrolled<10>([&](auto j) { pending |= !tail_ready(e[j], ep); });
            if (!pending) break;
            if (++spins == kTailSpinLimit) {
                atomicOr(T.table->status[s], HQ_STEP_SYNC);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
            unrolled<kSwigluTailB>([&](auto j) {
                if (!tail_ready(mb[j], ep)) mb[j] = tail_load(T.pmax + size_t(tid + kBlock * j) * p.m + s);
            });
            unrolled<10>([&](auto j) {
                if (!tail_ready(e[j], ep)) e[j] = tail_load(vsrc + i0 + kBlock * j);
            });
        }
        unrolled<kSwigluTailB>([&](auto j) {
            if (tid + kBlock * j < nb) mx = fmaxf(mx, bits_f32(uint32_t(mb[j])));
        });
        mx = wave_max64_all(mx);
        if (lane == 0) wmax[tid / kWave] = mx;
    }
    __syncthreads();
    if (on) {
        float amax = wmax[0];
#pragma unroll
        for (int w = 1; w < kBlock / kWave; ++w) amax = fmaxf(amax, wmax[w]);
        amax = fmaxf(amax, 1e-5f);
        const float inv = 127.0f / amax;
        unrolled<10>([&](auto j) {
            const int i = i0 + kBlock * j;
            if (i < n) T.q[bq_pos(s, xq_offset(i), T.kq)] = quant_i8(bits_f32(uint32_t(e[j])), inv);
        });
        if (qt == 0 && tid == 0) T.act[s] = amax / 127.0f;
    }
}

// The same products with the weight rows staged through LDS, for rows of up
// to HMAX packed bytes.  The block's R = 16 RG rows are one contiguous
// R * K/2 byte range of the matrix; its threads read it in 16-byte chunks,
// consecutive lanes taking consecutive chunks, so one wave instruction reads
// 1 KB of contiguous memory (an MFMA-shaped load -- 16 rows x 64 bytes --
// streams a 25 MB matrix in 7.2 us where contiguous 1 KB reads take 5.2 us).
// The chunks go to LDS rows padded by 16 bytes: the 16 rows of an A operand
// then start 4 banks apart, so the 16 lanes of a ds_read_b128 phase hit 64
// distinct banks.  Each wave's activation (B) loads go out with the weight
// loads; after one LDS barrier the wave runs the MFMAs of its double steps
// with A from LDS, and the int32 partial tiles meet in the same LDS.
// DS * W covers the double steps of any K up to 2 * HMAX (one round of B
// loads per wave), CPT * W * 64 chunks cover the block's rows.
template <int RG, int W, int BT, int DS, int CPT, int HMAX, bool SWIGLU, int TAIL>
__device__ __forceinline__ void gemm_lds_block(const GemmParams& p, uint8_t* a_s)
{
    static_assert(!SWIGLU || RG == 2, "a SwiGLU block pairs 16 gate rows with their 16 up rows");
    // TAIL: 0 (plain outputs), -1 ({value, epoch} entries in p.tail.ll, no
    // tail blocks) or, with entries and tail blocks, the values per thread
    // of a tail row (rows of up to 256 * TAIL; 1 for SwiGLU)
    static_assert(TAIL <= 0 || W >= 4, "a tail takes 256 threads of the block");
    constexpr int R = 16 * RG;
    constexpr int RS = HMAX + 16;                       // padded LDS row (bytes)
    constexpr int NRED = RG * BT * 4;                   // partial registers per lane
    static_assert(W * NRED * kWave * 4 <= R * RS, "the partial tiles alias the staged rows");
    static_assert(CPT * kWave * W * 16 >= R * HMAX, "the chunks of a thread cover the block's rows");
    static_assert(DS * W * 128 >= 2 * HMAX, "one round of B loads covers a wave's double steps");
    if constexpr (TAIL > 0) {
        // the launch's last blocks (after every tile's block, so each block
        // they wait for has started) only finish rows: one per row (o,
        // down) or four per row (gate_up)
        const int u = int(blockIdx.x) - tail_tiles<SWIGLU>(p);
        if (u >= 0) {   // (block-uniform)
            __shared__ float t_red[kBlock];
            __shared__ float t_wmax[kBlock / kWave];
            if constexpr (SWIGLU) gemm_swiglu_tail_row(p, u % p.m, u / p.m, tail_epoch(p.tail), t_wmax);
            else gemm_tail_row<TAIL>(p, u, tail_epoch(p.tail), t_red, t_wmax);
            return;
        }
    }
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid & (kWave - 1);
    const int q = lane >> 4;
    const int r16 = lane & 15;
    const int row0 = blockIdx.x * R;
    const int half = p.k >> 1;                          // packed bytes per row (a multiple of 16)
    const int cpr = half >> 4;                          // 16-byte chunks per row
    // Every load below is unconditional (clamped into range), so the
    // compiler tracks them by count: the LDS stores wait for the weight
    // chunks alone, and no branch splits the burst.  A chunk index past the
    // block's rows re-reads (and re-stores, to the same place) the last one.
    // SwiGLU: LDS rows 0-15 are gate rows 16b.., 16-31 the up rows n + 16b..
    // (two contiguous ranges); a row past n re-reads the last valid one.
    const int g0 = blockIdx.x * 16;
    const int ng = min(16, p.n - g0);                   // SwiGLU: valid rows per range
    const int total = SWIGLU ? R * cpr : min(R, p.n - row0) * cpr;
    const uint8_t* wb = p.w + size_t(row0) * size_t(half);
    auto chunk_addr = [&](int c) {
        if constexpr (SWIGLU) {
            const int r = int(unsigned(c) / unsigned(cpr));
            const int row = (r >= 16 ? p.n : 0) + g0 + min(r & 15, ng - 1);
            return p.w + size_t(row) * size_t(half) + size_t(c - r * cpr) * 16;
        } else {
            return wb + size_t(c) * 16;
        }
    };
    // SwiGLU in two stages: chunks j < CPT / 2 of a thread hold gate rows,
    // the rest up rows, and the activation loads go out between the two,
    // so the gate rows' MFMAs run while the up rows stream
    constexpr bool TWO = SWIGLU && (CPT % 2 == 0);
    static_assert(!TWO || (CPT / 2) * kWave * W * 16 >= 16 * HMAX, "half the chunks cover 16 rows");
    const int gcn = 16 * cpr;   // SwiGLU: the gate rows' chunks
    auto chunk_of = [&](int j) {
        if constexpr (TWO) {
            const int jj = j < CPT / 2 ? j : j - CPT / 2;
            return (j < CPT / 2 ? 0 : gcn) + min(tid + kWave * W * jj, gcn - 1);
        } else {
            return min(tid + kWave * W * j, total - 1);
        }
    };
    uint4 v[CPT];
#pragma unroll
    for (int j = 0; j < (TWO ? CPT / 2 : CPT); ++j) v[j] = load16_nt(chunk_addr(chunk_of(j)));
    const int nds = (p.k + 127) >> 7;
    const int ds0 = nds * wave / W, ds1 = nds * (wave + 1) / W;
    uint4 xb[DS][BT][2];
#pragma unroll
    for (int b = 0; b < BT; ++b) {
#pragma unroll
        for (int j = 0; j < DS; ++j) {
            // columns 2pb .. 2pb + 32 of a double step of row 16 b + r16
            // (bq_pos: 1 KB contiguous per wave load; rows past m re-read
            // row m - 1, whose lines the load fetches anyway, and land in
            // discarded columns; the MFMAs of the steps past the wave's
            // range are skipped)
            const int8_t* xp =
                p.x + bq_pos(min(16 * b + r16, p.m - 1), 2 * (min(ds0 + j, nds - 1) * 64 + 16 * q), p.kp);
            xb[j][b][0] = *reinterpret_cast<const uint4*>(xp);
            xb[j][b][1] = *reinterpret_cast<const uint4*>(xp + 1024);
        }
    }
    if constexpr (TWO) {
#pragma unroll
        for (int j = CPT / 2; j < CPT; ++j) v[j] = load16_nt(chunk_addr(chunk_of(j)));
    }
    // the epilogue's activation and row scales, fetched with the rest
    // (SwiGLU: element e = sequence e / 16, column e % 16 of the gate and up
    // tiles; the up row's scale in wu_e)
    constexpr int NE = SWIGLU ? 16 * 16 * BT : R * 16 * BT;
    constexpr int ER = SWIGLU ? 16 : R;
    constexpr int EPT = (NE + kWave * W - 1) / (kWave * W);
    float act_e[EPT], ws_e[EPT], wu_e[SWIGLU ? EPT : 1];
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const int e = tid + kWave * W * i;
        act_e[i] = p.act[min(e / ER, p.m - 1)];   // sequence e / ER, row e % ER
        if constexpr (SWIGLU) {
            ws_e[i] = p.ws[g0 + min(e % 16, ng - 1)];
            wu_e[i] = p.ws[p.n + g0 + min(e % 16, ng - 1)];
        } else {
            ws_e[i] = p.ws[min(row0 + e % R, p.n - 1)];
        }
    }
    auto stage = [&](int j0, int j1) {
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            if (j >= j0 && j < j1) {
                const int c = chunk_of(j);
                const int r = int(unsigned(c) / unsigned(cpr));
                *reinterpret_cast<uint4*>(a_s + r * RS + (c - r * cpr) * 16) = v[j];
            }
        }
        lds_sync();
    };
    stage(0, TWO ? CPT / 2 : CPT);

    i32x4 acc[RG][BT];
#pragma unroll
    for (int rg = 0; rg < RG; ++rg)
#pragma unroll
        for (int b = 0; b < BT; ++b) acc[rg][b] = i32x4{0, 0, 0, 0};
    constexpr uint32_t m4 = 0xF0F0F0F0u;
    // the MFMAs of row groups [rg0, rg1) over the wave's double steps
    auto products = [&](int rg0, int rg1) {
#pragma unroll
        for (int j = 0; j < DS; ++j) {
            const int pb = (ds0 + j) * 64 + 16 * q;        // this lane's 16 packed bytes of the row
            if (ds0 + j < ds1) {
#pragma unroll
                for (int rg = 0; rg < RG; ++rg) {
                    if (rg < rg0 || rg >= rg1) continue;
                    // past K the activations are zero, so the padding read there adds 0
                    const uint4 w = pb < half ? *reinterpret_cast<const uint4*>(a_s + (16 * rg + r16) * RS + pb)
                                              : make_uint4(0, 0, 0, 0);
                    const i32x4 a0 = {int((w.x << 4) & m4), int(w.x & m4), int((w.y << 4) & m4), int(w.y & m4)};
                    const i32x4 a1 = {int((w.z << 4) & m4), int(w.z & m4), int((w.w << 4) & m4), int(w.w & m4)};
#pragma unroll
                    for (int b = 0; b < BT; ++b) {
                        const uint4 x0 = xb[j][b][0], x1 = xb[j][b][1];
                        acc[rg][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            a0, i32x4{int(x0.x), int(x0.y), int(x0.z), int(x0.w)}, acc[rg][b], 0, 0, 0);
                        acc[rg][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            a1, i32x4{int(x1.x), int(x1.y), int(x1.z), int(x1.w)}, acc[rg][b], 0, 0, 0);
                    }
                }
            }
        }
    };
    if constexpr (TWO) {
        products(0, 1);         // gate rows (LDS rows 0-15), while the up rows stream
        stage(CPT / 2, CPT);    // (the up rows go to LDS rows 16-31)
        products(1, 2);
    } else {
        products(0, RG);
    }
    lds_sync();   // every wave's A reads are done: the partials reuse the LDS
    int32_t (*red)[NRED][kWave] = reinterpret_cast<int32_t (*)[NRED][kWave]>(a_s);
#pragma unroll
    for (int rg = 0; rg < RG; ++rg)
#pragma unroll
        for (int b = 0; b < BT; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][(rg * BT + b) * 4 + r][lane] = acc[rg][b][r];
    lds_sync();
    const uint32_t ep = TAIL != 0 ? tail_epoch(p.tail) : 0u;
    if constexpr (SWIGLU) {
        // element e: sequence e / 16, column e % 16 of the gate and up tiles;
        // the 16 columns of a sequence sit in one 16-lane row of a wave
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            const int e = tid + kWave * W * i;
            if (e >= NE) break;
            const int rr = e & 15, ml = e >> 4;
            const int b = ml >> 4, col = ml & 15;
            const int src = col + 16 * (rr >> 2);
            const int regg = b * 4 + (rr & 3), regu = (BT + b) * 4 + (rr & 3);
            int32_t sg = 0, su = 0;
#pragma unroll
            for (int w2 = 0; w2 < W; ++w2) {
                sg += red[w2][regg][src];
                su += red[w2][regu][src];
            }
            const float g = (float(sg >> 4) * act_e[i]) * ws_e[i];
            const float u = (float(su >> 4) * act_e[i]) * wu_e[i];
            const float t = 1.0f + spec_expf(-g);
            const float v = (g / t) * u;
            const bool ok = ml < p.m && rr < ng;
            if (ok) {
                if constexpr (TAIL != 0) tail_store(p.tail.ll + size_t(ml) * p.n + g0 + rr, v, ep);
                else p.out[size_t(ml) * p.n + g0 + rr] = v;
            }
            float mx = ok ? fabsf(v) : 0.0f;
#pragma unroll
            for (int o = 8; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 16));
            if (rr == 0 && ml < p.m) {
                if constexpr (TAIL != 0) tail_store(p.tail.pmax + size_t(blockIdx.x) * p.m + ml, mx, ep);
                else p.pmax[size_t(blockIdx.x) * p.m + ml] = mx;
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            const int e = tid + kWave * W * i;
            if (e >= NE) break;
            const int rl = e % R, ml = e / R;
            const int rg = rl >> 4, rr = rl & 15, b = ml >> 4, col = ml & 15;
            const int src = col + 16 * (rr >> 2), reg = (rg * BT + b) * 4 + (rr & 3);
            int32_t sum = 0;
#pragma unroll
            for (int w2 = 0; w2 < W; ++w2) sum += red[w2][reg][src];
            const int mm = 16 * b + col, n = row0 + rl;
            if (mm < p.m && n < p.n) {
                const int a = sum >> 4;
                const float v = (float(a) * act_e[i]) * ws_e[i];
                if constexpr (TAIL != 0) {
                    __hip_atomic_store(p.tail.ll + size_t(mm) * p.n + n, (uint64_t(ep) << 32) | uint64_t(f32_bits(v)),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                } else {
                    p.out[size_t(mm) * p.n + n] = v;
                    if (p.acc_out) p.acc_out[size_t(mm) * p.n + n] = a;
                }
            }
        }
    }
}

}  // namespace hq
