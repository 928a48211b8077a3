// hq_gemm.hip - batched decode: packed-int4 weights x M int8 activation
// vectors on gfx950 int8 MFMA (v_mfma_i32_16x16x64_i8).
//
// The reference decodes one sequence at a time (cpu_lightspark.py:424 in the
// reference repository); M sequences are defined as M independent GEMVs of
// cpu_kernels/litespark_int4.cpp:22-76, and this kernel returns exactly
// those integers: out[m,n] = ((float)acc[m,n] * act[m]) * scale[n].
//
// Mapping onto the MFMA: weight rows go on the 16-row A side, the batch on
// the 16-column B side (M = 8 fills half of B; M = 32 uses two B tiles).
// A lane of the A operand carries 16 K values of one weight row; the nibbles
// of a packed dword become signed bytes (w << 4) & 0xF0F0F0F0 (16 * even
// columns) and w & 0xF0F0F0F0 (16 * odd columns), so the MFMA accumulates
// 16 * acc exactly.  The B operand is the activations in the same per-8-column
// even/odd order (the quantizing kernels write them so, rows padded with
// zeros to whole 256-column slices), read straight from global memory (L2):
// lane group q of a "double step" of 128 columns holds columns [32q, 32q+32)
// as two 16-column MFMA operands, for A from one 16-byte load of the packed
// row and for B from two 16-byte loads of the activation row.
//
// A block owns RG groups of 16 rows over the whole K; its W waves split K
// (each a contiguous range of double steps, all of its loads in flight at
// once) and their int32 partial tiles meet in LDS, so no split of K crosses
// blocks: no atomics, no arrival tickets, no zeroed workspace.
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

template <int RG, int W, int BT, int DS>
__global__ __launch_bounds__(kWave * W) void gemm_kernel(GemmParams p)
{
    __shared__ int32_t red[W][RG * BT * 4][kWave];
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid & (kWave - 1);
    const int q = lane >> 4;                    // lane group: columns [32q, 32q + 32) of a double step
    const int r16 = lane & 15;                  // A: row within a group; B: sequence within a tile
    const int row0 = blockIdx.x * 16 * RG;
    const int half = p.k >> 1;                  // packed bytes per row (a multiple of 16)
    const int nds = (p.k + 127) >> 7;           // double steps of 128 columns
    const int ds0 = nds * wave / W, ds1 = nds * (wave + 1) / W;
    const uint8_t* arow[RG];
    bool aok[RG];
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
        const int row = row0 + 16 * rg + r16;
        aok[rg] = row < p.n;
        arow[rg] = p.w + size_t(aok[rg] ? row : 0) * size_t(half);
    }
    const int8_t* brow[BT];
#pragma unroll
    for (int b = 0; b < BT; ++b) brow[b] = p.x + size_t(min(16 * b + r16, p.m - 1)) * size_t(p.kp);

    i32x4 acc[RG][BT];
#pragma unroll
    for (int rg = 0; rg < RG; ++rg)
#pragma unroll
        for (int b = 0; b < BT; ++b) acc[rg][b] = i32x4{0, 0, 0, 0};
    constexpr uint32_t m4 = 0xF0F0F0F0u;
    for (int d0 = ds0; d0 < ds1; d0 += DS) {
        const int nd = min(DS, ds1 - d0);
        uint4 wa[DS][RG], xb[DS][BT][2];
#pragma unroll
        for (int j = 0; j < DS; ++j) {
            const int pb = (d0 + j) * 64 + 16 * q;          // this lane's 16 packed bytes
#pragma unroll
            for (int rg = 0; rg < RG; ++rg)
                wa[j][rg] = (j < nd && aok[rg] && pb < half)
                                ? load16_nt(arow[rg] + pb)
                                : make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int b = 0; b < BT; ++b) {
                const int8_t* xp = brow[b] + 2 * pb;             // columns 2pb .. 2pb + 32 (zero past K)
                xb[j][b][0] = j < nd ? *reinterpret_cast<const uint4*>(xp) : make_uint4(0, 0, 0, 0);
                xb[j][b][1] = j < nd ? *reinterpret_cast<const uint4*>(xp + 16) : make_uint4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int j = 0; j < DS; ++j) {
            if (j < nd) {
#pragma unroll
                for (int rg = 0; rg < RG; ++rg) {
                    const uint4 w = wa[j][rg];
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
    }
    // D layout: lane holds rows 4 * (lane / 16) + r, column lane % 16
#pragma unroll
    for (int rg = 0; rg < RG; ++rg)
#pragma unroll
        for (int b = 0; b < BT; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][(rg * BT + b) * 4 + r][lane] = acc[rg][b][r];
    __syncthreads();
    // element e of the block's (16 RG rows) x (16 BT sequences) tile: rows
    // fastest, so the stores of one sequence are contiguous
    constexpr int NR = 16 * RG;
    for (int e = tid; e < NR * 16 * BT; e += kWave * W) {
        const int rl = e % NR, ml = e / NR;
        const int rg = rl >> 4, rr = rl & 15, b = ml >> 4, col = ml & 15;
        const int src = col + 16 * (rr >> 2), reg = (rg * BT + b) * 4 + (rr & 3);
        int32_t sum = 0;
#pragma unroll
        for (int w2 = 0; w2 < W; ++w2) sum += red[w2][reg][src];
        const int mm = 16 * b + col, n = row0 + rl;
        if (mm < p.m && n < p.n) {
            const int a = sum >> 4;
            p.out[size_t(mm) * p.n + n] = (float(a) * p.act[mm]) * p.ws[n];
            if (p.acc_out) p.acc_out[size_t(mm) * p.n + n] = a;
        }
    }
}

// ---- batched-step tails ------------------------------------------------------------

__device__ __forceinline__ uint32_t tail_epoch(const GemmTail& t)
{
    return (*t.epoch_ctr << 8) | uint32_t(t.epoch_id);
}


// Row s of a tail launch, by threads 0-255 of one block (the others only
// take the barriers): once every block's entry of the row is current (each
// block stores its outputs before its tail begins; blocks start in index
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
        int8_t* qr = T.q + size_t(s) * T.kq;
#pragma unroll
        for (int j = 0; j < NPT; ++j) {
            const int i = tid + kBlock * j;
            if (i < k) qr[xq_offset(i)] = quant_i8(v[j], inv);
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
__device__ void gemm_swiglu_tail_row(const GemmParams& p, int s, int qt, uint32_t ep, float* wmax)
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
        int8_t* qr = T.q + size_t(s) * T.kq;
        unrolled<10>([&](auto j) {
            const int i = i0 + kBlock * j;
            if (i < n) qr[xq_offset(i)] = quant_i8(bits_f32(uint32_t(e[j])), inv);
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
template <int RG, int W, int BT, int DS, int CPT, int HMAX, bool SWIGLU = false, int TAIL = 0>
__global__ __launch_bounds__(kWave * W) void gemm_lds_kernel(GemmParams p)
{
    static_assert(!SWIGLU || RG == 2, "a SwiGLU block pairs 16 gate rows with their 16 up rows");
    // TAIL: 0, or the values per thread of a tail row (rows of up to 256 * TAIL)
    static_assert(!TAIL || W >= 4, "a tail takes 256 threads of the block");
    constexpr int R = 16 * RG;
    constexpr int RS = HMAX + 16;                       // padded LDS row (bytes)
    constexpr int NRED = RG * BT * 4;                   // partial registers per lane
    static_assert(W * NRED * kWave * 4 <= R * RS, "the partial tiles alias the staged rows");
    static_assert(CPT * kWave * W * 16 >= R * HMAX, "the chunks of a thread cover the block's rows");
    static_assert(DS * W * 128 >= 2 * HMAX, "one round of B loads covers a wave's double steps");
    __shared__ __align__(16) uint8_t a_s[R * RS];
    if constexpr (TAIL) {
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
    uint4 v[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) v[j] = load16_nt(chunk_addr(min(tid + kWave * W * j, total - 1)));
    const int nds = (p.k + 127) >> 7;
    const int ds0 = nds * wave / W, ds1 = nds * (wave + 1) / W;
    uint4 xb[DS][BT][2];
#pragma unroll
    for (int b = 0; b < BT; ++b) {
        const int8_t* brow = p.x + size_t(min(16 * b + r16, p.m - 1)) * size_t(p.kp);
#pragma unroll
        for (int j = 0; j < DS; ++j) {
            // columns 2pb .. 2pb + 32 of a double step inside the row (the
            // MFMAs of the steps past the wave's range are skipped)
            const int8_t* xp = brow + 2 * (min(ds0 + j, nds - 1) * 64 + 16 * q);
            xb[j][b][0] = *reinterpret_cast<const uint4*>(xp);
            xb[j][b][1] = *reinterpret_cast<const uint4*>(xp + 16);
        }
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
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int c = min(tid + kWave * W * j, total - 1);
        const int r = int(unsigned(c) / unsigned(cpr));
        *reinterpret_cast<uint4*>(a_s + r * RS + (c - r * cpr) * 16) = v[j];
    }
    lds_sync();

    i32x4 acc[RG][BT];
#pragma unroll
    for (int rg = 0; rg < RG; ++rg)
#pragma unroll
        for (int b = 0; b < BT; ++b) acc[rg][b] = i32x4{0, 0, 0, 0};
    constexpr uint32_t m4 = 0xF0F0F0F0u;
#pragma unroll
    for (int j = 0; j < DS; ++j) {
        const int pb = (ds0 + j) * 64 + 16 * q;        // this lane's 16 packed bytes of the row
        if (ds0 + j < ds1) {
#pragma unroll
            for (int rg = 0; rg < RG; ++rg) {
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
    lds_sync();   // every wave's A reads are done: the partials reuse the LDS
    int32_t (*red)[NRED][kWave] = reinterpret_cast<int32_t (*)[NRED][kWave]>(a_s);
#pragma unroll
    for (int rg = 0; rg < RG; ++rg)
#pragma unroll
        for (int b = 0; b < BT; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][(rg * BT + b) * 4 + r][lane] = acc[rg][b][r];
    lds_sync();
    const uint32_t ep = TAIL ? tail_epoch(p.tail) : 0u;
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
                if constexpr (TAIL) tail_store(p.tail.ll + size_t(ml) * p.n + g0 + rr, v, ep);
                else p.out[size_t(ml) * p.n + g0 + rr] = v;
            }
            float mx = ok ? fabsf(v) : 0.0f;
#pragma unroll
            for (int o = 8; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 16));
            if (rr == 0 && ml < p.m) {
                if constexpr (TAIL) tail_store(p.tail.pmax + size_t(blockIdx.x) * p.m + ml, mx, ep);
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
                if constexpr (TAIL) {
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

// The batched step's down input: block m (1024 threads) takes sequence m's
// SwiGLU row (gemm_lds_kernel's SwiGLU output), its maximum |value| from the
// GEMM blocks' partial maxima (order-free), and quantizes it as the SwiGLU
// row kernel does (amax floored at 1e-5, quant_i8 with 127 / amax, columns
// de-interleaved per 8, row stride kp), with amax / 127 in act[m].
constexpr int kActQuantThreads = 1024;
constexpr int kActQuantNPT = 10;     // rows of up to 10240 values
__global__ __launch_bounds__(kActQuantThreads) void batch_act_quant_kernel(const float* a, const float* pmax,
                                                                            int nblocks, int m_count, int n, int kp,
                                                                            int8_t* q, float* act)
{
    __shared__ float wred[kActQuantThreads / kWave];
    const int m = blockIdx.x;
    const int t = threadIdx.x;
    const float* row = a + size_t(m) * n;
    float v[kActQuantNPT];
#pragma unroll
    for (int j = 0; j < kActQuantNPT; ++j) {
        const int i = t + kActQuantThreads * j;
        v[j] = i < n ? row[i] : 0.0f;
    }
    float mx = 0.0f;
    for (int b = t; b < nblocks; b += kActQuantThreads) mx = fmaxf(mx, pmax[size_t(b) * m_count + m]);
    mx = wave_max64_all(mx);
    if ((t & (kWave - 1)) == 0) wred[t / kWave] = mx;
    lds_sync();
    float amax = wred[0];
#pragma unroll
    for (int w = 1; w < kActQuantThreads / kWave; ++w) amax = fmaxf(amax, wred[w]);
    amax = fmaxf(amax, 1e-5f);
    const float inv = 127.0f / amax;
    int8_t* qr = q + size_t(m) * kp;
#pragma unroll
    for (int j = 0; j < kActQuantNPT; ++j) {
        const int i = t + kActQuantThreads * j;
        if (i < n) qr[(i & ~7) + ((i & 1) ? 4 + ((i & 7) >> 1) : ((i & 7) >> 1))] = quant_i8(v[j], inv);
    }
    if (t == 0) act[m] = amax / 127.0f;
}

// Per-sequence spec quantization: block m quantizes row m into q (row
// stride kp, de-interleaved per 8 columns: the 4 even columns, then the 4
// odd ones) and, when given, q_out (natural order).  Thread t handles the
// 8-column groups t + 256i; every load is issued before any is used, so a
// row costs one memory round trip.
constexpr int kQuantGroups = 5;   // 8-column groups per thread: K <= 10240
__global__ __launch_bounds__(kBlock) void batch_quant_kernel(const float* x, int k, int kp, int8_t* q,
                                                             float* act, int8_t* q_out,
                                                             float* act_out)
{
    __shared__ float red[4];
    const int m = blockIdx.x;
    const float* xr = x + size_t(m) * k;
    const int t = threadIdx.x;
    float4 v[2 * kQuantGroups];
#pragma unroll
    for (int i = 0; i < kQuantGroups; ++i) {
        const int c = 8 * (t + kBlock * i);
        const bool ok = c < k;
        v[2 * i] = ok ? *reinterpret_cast<const float4*>(xr + c) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        v[2 * i + 1] = ok ? *reinterpret_cast<const float4*>(xr + c + 4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 2 * kQuantGroups; ++i)
        amax = fmaxf(fmaxf(amax, fmaxf(fabsf(v[i].x), fabsf(v[i].y))), fmaxf(fabsf(v[i].z), fabsf(v[i].w)));
    amax = block_max_nonneg(amax, red);
    amax = fmaxf(amax, 1e-5f);
    const float inv = 127.0f / amax;
    auto b8 = [&](float f) { return uint32_t(uint8_t(quant_i8(f, inv))); };
#pragma unroll
    for (int i = 0; i < kQuantGroups; ++i) {
        const int c = 8 * (t + kBlock * i);
        if (c < k) {
            const float4 a = v[2 * i], b = v[2 * i + 1];
            const uint32_t ev = b8(a.x) | (b8(a.z) << 8) | (b8(b.x) << 16) | (b8(b.z) << 24);
            const uint32_t od = b8(a.y) | (b8(a.w) << 8) | (b8(b.y) << 16) | (b8(b.w) << 24);
            *reinterpret_cast<uint2*>(q + size_t(m) * kp + c) = make_uint2(ev, od);
            if (q_out) {
                const uint32_t lo = b8(a.x) | (b8(a.y) << 8) | (b8(a.z) << 16) | (b8(a.w) << 24);
                const uint32_t hi = b8(b.x) | (b8(b.y) << 8) | (b8(b.z) << 16) | (b8(b.w) << 24);
                *reinterpret_cast<uint2*>(q_out + size_t(m) * k + c) = make_uint2(lo, hi);
            }
        }
    }
    if (t == 0) {
        act[m] = amax / 127.0f;
        if (act_out) act_out[m] = amax / 127.0f;
    }
}

// int8 activations in natural order -> the GEMM's de-interleaved padded rows
// (block m: row m).
__global__ __launch_bounds__(kBlock) void batch_deinterleave_kernel(const int8_t* x, int k, int kp, int8_t* q)
{
    const int m = blockIdx.x;
    for (int c = 8 * threadIdx.x; c < k; c += 8 * kBlock) {
        const uint2 v = *reinterpret_cast<const uint2*>(x + size_t(m) * k + c);
        uint32_t ev, od;
        deinterleave8(v.x, v.y, ev, od);
        *reinterpret_cast<uint2*>(q + size_t(m) * kp + c) = make_uint2(ev, od);
    }
}

struct GemmLayout {
    size_t q_off, act_off, total;
};

static size_t al256(size_t v) { return (v + 255) & ~size_t(255); }

static int padded_k(int k) { return (k + kSlice - 1) / kSlice * kSlice; }
static int padded_m(int m) { return (m + kMaxBatch - 1) / kMaxBatch * kMaxBatch; }

// The standalone entries' workspace: the de-interleaved padded activations
// (padded_m(m) rows of padded_k(k) bytes; padding bytes are never written,
// zero from the initial fill), then the activation scales.
static GemmLayout gemm_layout(int m, int n, int k)
{
    (void)n;
    GemmLayout L{};
    L.q_off = 0;
    L.act_off = al256(size_t(padded_m(m)) * size_t(padded_k(k)));
    L.total = L.act_off + al256(size_t(m) * 4);
    return L;
}

template <int RG, int W, int BT>
static void launch_gemm(const GemmParams& p, hipStream_t s)
{
    // double steps one wave keeps in flight: all of its range up to K =
    // W * DS * 128 (a 1024-thread block holds fewer registers per lane, the
    // more so with two sequence tiles)
    constexpr int DS = W == 16 ? (BT == 2 ? 4 : 5) : 6;
    hipLaunchKernelGGL((gemm_kernel<RG, W, BT, DS>), dim3((p.n + 16 * RG - 1) / (16 * RG)), dim3(kWave * W), 0, s,
                       p);
}

template <int RG, int W, int BT, int HMAX>
static void launch_gemm_lds(const GemmParams& p, hipStream_t s)
{
    constexpr int R = 16 * RG;
    constexpr int DS = (2 * HMAX / 128 + W - 1) / W;
    constexpr int CPT = (R * HMAX / 16 + kWave * W - 1) / (kWave * W);
    hipLaunchKernelGGL((gemm_lds_kernel<RG, W, BT, DS, CPT, HMAX>), dim3((p.n + R - 1) / R), dim3(kWave * W), 0, s,
                       p);
}

// Rows of up to 5120 packed bytes (K <= 10240) take the LDS-staged kernel:
// 4 waves per block up to K = 2560, 8 up to 4096, 16 beyond; 32 rows per
// block up to K = 2560 for two sequence tiles, and for one over 2048 blocks
// or more (the LM head: 43.2 against 47.8 us at M = 8, where gate_up's 608
// blocks of 32 rows took 11.2 against 10.4 us for 1216 of 16).
template <int BT>
static bool launch_staged(const GemmParams& p, bool two_groups, hipStream_t s)
{
    const int half = p.k >> 1;
    if (half <= 1280) {
        // two sequence tiles share each weight row over 32 rows (M = 32:
        // gate_up 18.8 -> 16.9 us, the LM head 106.8 -> 81.7 us)
        if (two_groups || BT == 2) launch_gemm_lds<2, 4, BT, 1280>(p, s);
        else launch_gemm_lds<1, 4, BT, 1280>(p, s);
    } else if (half <= 2048) {
        launch_gemm_lds<1, 8, BT, 2048>(p, s);
    } else if (half <= 5120) {
        launch_gemm_lds<1, 16, BT, 5120>(p, s);
    } else {
        return false;
    }
    return true;
}

// x: the de-interleaved padded activations.  Wider rows: the kernel with
// MFMA-shaped weight loads; waves per block: the fewest of 4, 8, 16 whose K
// ranges fit one round of loads; 32 rows per block from 512 blocks up.
static hipError_t run_gemm(const int8_t* x, const float* act, const uint8_t* w, const float* ws,
                           float* out, int m, int n, int k, int32_t* acc_out, hipStream_t s)
{
    const int kp = padded_k(k);
    const int nds = (k + 127) / 128;
    const int waves = nds <= 4 * 6 ? 4 : nds <= 8 * 6 ? 8 : 16;
    for (int m0 = 0; m0 < m; m0 += kMaxBatch) {
        GemmParams p{};
        p.m = m - m0 < kMaxBatch ? m - m0 : kMaxBatch;
        p.x = x + size_t(m0) * kp;
        p.act = act + m0;
        p.w = w; p.ws = ws;
        p.out = out + size_t(m0) * n;
        p.acc_out = acc_out ? acc_out + size_t(m0) * n : nullptr;
        p.n = n; p.k = k; p.kp = kp;
        const bool two_groups = p.m <= 16 && (n + 31) / 32 >= ((k >> 1) <= 5120 ? 2048 : 512);
        const bool staged = p.m > 16 ? launch_staged<2>(p, two_groups, s) : launch_staged<1>(p, two_groups, s);
        if (staged) {
        } else if (p.m > 16) {
            if (waves == 4) launch_gemm<1, 4, 2>(p, s);
            else if (waves == 8) launch_gemm<1, 8, 2>(p, s);
            else launch_gemm<1, 16, 2>(p, s);
        } else if (two_groups) {
            if (waves == 4) launch_gemm<2, 4, 1>(p, s);
            else if (waves == 8) launch_gemm<2, 8, 1>(p, s);
            else launch_gemm<2, 16, 1>(p, s);
        } else {
            if (waves == 4) launch_gemm<1, 4, 1>(p, s);
            else if (waves == 8) launch_gemm<1, 8, 1>(p, s);
            else launch_gemm<1, 16, 1>(p, s);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int W, int BT, int HMAX>
static void launch_swiglu(const GemmParams& p, hipStream_t s)
{
    constexpr int DS = (2 * HMAX / 128 + W - 1) / W;
    constexpr int CPT = (32 * HMAX / 16 + kWave * W - 1) / (kWave * W);
    hipLaunchKernelGGL((gemm_lds_kernel<2, W, BT, DS, CPT, HMAX, true>), dim3((p.n + 15) / 16), dim3(kWave * W), 0,
                       s, p);
}

int gemm_swiglu_blocks(int n) { return (n + 15) / 16; }

template <int W, int BT, int HMAX>
static void launch_swiglu_tail(const GemmParams& p, hipStream_t s)
{
    constexpr int DS = (2 * HMAX / 128 + W - 1) / W;
    constexpr int CPT = (32 * HMAX / 16 + kWave * W - 1) / (kWave * W);
    hipLaunchKernelGGL((gemm_lds_kernel<2, W, BT, DS, CPT, HMAX, true, 1>), dim3((p.n + 15) / 16 + 4 * p.m),
                       dim3(kWave * W), 0, s, p);
}

template <int W, int BT, int HMAX>
static void launch_tail(const GemmParams& p, hipStream_t s)
{
    constexpr int DS = (2 * HMAX / 128 + W - 1) / W;
    constexpr int CPT = (16 * HMAX / 16 + kWave * W - 1) / (kWave * W);
    hipLaunchKernelGGL((gemm_lds_kernel<1, W, BT, DS, CPT, HMAX, false, kTailNPT>), dim3((p.n + 15) / 16 + p.m),
                       dim3(kWave * W), 0, s, p);
}

bool gemm_tail_fits(int m, int n, int k)
{
    const int half = k >> 1;
    return m >= 1 && m <= kMaxBatch && n <= kBlock * kTailNPT && (n + 15) / 16 >= m && half > 1280 &&
           half <= 5120;
}

// The batched step's o and down GEMMs with the residual + RMSNorm + quant
// rows of the next GEMM's input in their tail (see GemmParams::tail).
hipError_t gemm_run_tail(const int8_t* x, const float* act, const uint8_t* w, const float* ws, int m, int n, int k,
                         const GemmTail& tail, hipStream_t s)
{
    if (!gemm_tail_fits(m, n, k) || tail.epoch_id < 0 || tail.epoch_id >= 256) return hipErrorInvalidValue;
    GemmParams p{};
    p.m = m;
    p.x = x;
    p.act = act;
    p.w = w; p.ws = ws;
    p.n = n; p.k = k; p.kp = padded_k(k);
    p.tail = tail;
    const int half = k >> 1;
    if (half <= 2048) {
        if (m > 16) launch_tail<8, 2, 2048>(p, s);
        else launch_tail<8, 1, 2048>(p, s);
    } else {
        if (m > 16) launch_tail<16, 2, 5120>(p, s);
        else launch_tail<16, 1, 5120>(p, s);
    }
    return hipGetLastError();
}

// gate_up with SwiGLU in the GEMM epilogue, then the down input's
// quantization: act_out [m, n] fp32, q [m, kq] int8 + act [m].
hipError_t gemm_run_swiglu(const int8_t* x, const float* act, const uint8_t* w, const float* ws, float* act_out,
                           int m, int n, int k, float* pmax, int8_t* q, int kq, float* act_q, hipStream_t s)
{
    if (m < 1 || m > kMaxBatch || (k >> 1) > 2048 || n > kActQuantThreads * kActQuantNPT || !pmax)
        return hipErrorInvalidValue;
    GemmParams p{};
    p.m = m;
    p.x = x;
    p.act = act;
    p.w = w; p.ws = ws;
    p.out = act_out;
    p.n = n; p.k = k; p.kp = padded_k(k);
    p.pmax = pmax;
    if ((k >> 1) <= 1280) {
        if (m > 16) launch_swiglu<4, 2, 1280>(p, s);
        else launch_swiglu<4, 1, 1280>(p, s);
    } else {
        if (m > 16) launch_swiglu<8, 2, 2048>(p, s);
        else launch_swiglu<8, 1, 2048>(p, s);
    }
    hipLaunchKernelGGL(batch_act_quant_kernel, dim3(m), dim3(kActQuantThreads), 0, s, act_out, pmax,
                       gemm_swiglu_blocks(n), m, n, kq, q, act_q);
    return hipGetLastError();
}

bool gemm_swiglu_tail_fits(int m, int n, int k)
{
    return m >= 1 && m <= kMaxBatch && (k >> 1) <= 2048 && n <= 4 * kSwigluTailQ &&
           gemm_swiglu_blocks(n) <= kBlock * kSwigluTailB && gemm_swiglu_blocks(n) >= 4 * m;
}

// gate_up with SwiGLU in the epilogue and the down input's quantization in
// the tail (see GemmParams::tail; tail.ll holds [m, n] entries, tail.pmax
// gemm_swiglu_blocks(n) * m).
hipError_t gemm_run_swiglu_tail(const int8_t* x, const float* act, const uint8_t* w, const float* ws, int m, int n,
                                int k, const GemmTail& tail, hipStream_t s)
{
    if (!gemm_swiglu_tail_fits(m, n, k) || tail.epoch_id < 0 || tail.epoch_id >= 256) return hipErrorInvalidValue;
    GemmParams p{};
    p.m = m;
    p.x = x;
    p.act = act;
    p.w = w; p.ws = ws;
    p.n = n; p.k = k; p.kp = padded_k(k);
    p.tail = tail;
    if ((k >> 1) <= 1280) {
        if (m > 16) launch_swiglu_tail<4, 2, 1280>(p, s);
        else launch_swiglu_tail<4, 1, 1280>(p, s);
    } else {
        if (m > 16) launch_swiglu_tail<8, 2, 2048>(p, s);
        else launch_swiglu_tail<8, 1, 2048>(p, s);
    }
    return hipGetLastError();
}

int gemm_padded_k(int k) { return padded_k(k); }
int gemm_padded_m(int m) { return padded_m(m); }
size_t gemm_scratch_bytes(int m, int n, int k)
{
    (void)m; (void)n; (void)k;
    return 0;   // the GEMM itself needs no workspace
}
hipError_t gemm_run(const int8_t* x, const float* act, const uint8_t* w, const float* ws, float* out, int m, int n,
                    int k, char* scratch, hipStream_t s)
{
    (void)scratch;
    return run_gemm(x, act, w, ws, out, m, n, k, nullptr, s);
}

}  // namespace hq

using namespace hq;

extern "C" size_t hq_gemm_workspace_bytes(int m, int rows, int width)
{
    if (m <= 0 || rows <= 0 || width <= 0) return 0;
    return gemm_layout(m, rows, width).total;
}

extern "C" int hq_int4_i8_gemm(const int8_t* x, const float* act_scales, const uint8_t* weights,
                               const float* scales, float* output, int m, int rows, int width,
                               int32_t* acc_out, void* workspace, void* stream)
{
    if (m <= 0 || rows < 0 || width <= 0 || (width & 31)) return HQ_ERR_ARG;
    if (rows == 0) return HQ_OK;
    if (!x || !act_scales || !weights || !scales || !output || !workspace) return HQ_ERR_ARG;
    if (!al16(weights) || !al16(x) || !al16(workspace)) return HQ_ERR_ALIGN;
    hipStream_t s = static_cast<hipStream_t>(stream);
    char* ws = static_cast<char*>(workspace);
    const GemmLayout L = gemm_layout(m, rows, width);
    int8_t* q = reinterpret_cast<int8_t*>(ws + L.q_off);
    hipLaunchKernelGGL(batch_deinterleave_kernel, dim3(m), dim3(kBlock), 0, s, x, width, padded_k(width), q);
    if (hipGetLastError() != hipSuccess) return HQ_ERR_LAUNCH;
    const hipError_t e = run_gemm(q, act_scales, weights, scales, output, m, rows, width, acc_out, s);
    return e == hipSuccess ? HQ_OK : HQ_ERR_LAUNCH;
}

extern "C" int hq_quant_int4_gemm(const float* x, const uint8_t* weights, const float* scales,
                                  float* output, int m, int rows, int width, int8_t* q_out,
                                  float* act_scales_out, int32_t* acc_out, void* workspace,
                                  void* stream)
{
    if (m <= 0 || rows < 0 || width <= 0 || (width & 31) || width > 8 * kBlock * kQuantGroups) return HQ_ERR_ARG;
    if (rows == 0) return HQ_OK;
    if (!x || !weights || !scales || !output || !workspace) return HQ_ERR_ARG;
    if (!al16(weights) || !al16(workspace) || !al16(x)) return HQ_ERR_ALIGN;
    if (q_out && (reinterpret_cast<uintptr_t>(q_out) & 7u)) return HQ_ERR_ALIGN;
    hipStream_t s = static_cast<hipStream_t>(stream);
    char* ws = static_cast<char*>(workspace);
    const GemmLayout L = gemm_layout(m, rows, width);
    int8_t* q = reinterpret_cast<int8_t*>(ws + L.q_off);
    float* act = reinterpret_cast<float*>(ws + L.act_off);
    hipLaunchKernelGGL(batch_quant_kernel, dim3(m), dim3(kBlock), 0, s, x, width, padded_k(width), q, act,
                       q_out, act_scales_out);
    if (hipGetLastError() != hipSuccess) return HQ_ERR_LAUNCH;
    const hipError_t e = run_gemm(q, act, weights, scales, output, m, rows, width, acc_out, s);
    return e == hipSuccess ? HQ_OK : HQ_ERR_LAUNCH;
}
