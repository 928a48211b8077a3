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
// blocks: no atomics, no arrival tickets, no zeroed workspace.  (The
// batched decode step's launches with tails hand their outputs to extra
// blocks through {value, epoch} entries in its workspace: hq_gemm_block.h.)
#include "hq_gemm_block.h"

namespace hq {

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
                // columns 2pb .. 2pb + 32 of row 16 b + r16 (zero past K; bq_pos;
                // rows past m re-read row m - 1)
                const int8_t* xp = p.x + bq_pos(min(16 * b + r16, p.m - 1), 2 * pb, p.kp);
                xb[j][b][0] = j < nd ? *reinterpret_cast<const uint4*>(xp) : make_uint4(0, 0, 0, 0);
                xb[j][b][1] = j < nd ? *reinterpret_cast<const uint4*>(xp + 1024) : make_uint4(0, 0, 0, 0);
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

template <int RG, int W, int BT, int DS, int CPT, int HMAX, bool SWIGLU = false, int TAIL = 0>
__global__ __launch_bounds__(kWave * W, (W == 4 && BT == 2) ? 3 : 1) void gemm_lds_kernel(GemmParams p)
{
    __shared__ __align__(16) uint8_t a_s[16 * RG * (HMAX + 16)];
    gemm_lds_block<RG, W, BT, DS, CPT, HMAX, SWIGLU, TAIL>(p, a_s);
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
#pragma unroll
    for (int j = 0; j < kActQuantNPT; ++j) {
        const int i = t + kActQuantThreads * j;
        if (i < n) q[bq_pos(m, xq_offset(i), kp)] = quant_i8(v[j], inv);
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
            *reinterpret_cast<uint2*>(q + bq_pos(m, c, kp)) = make_uint2(ev, od);
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
        *reinterpret_cast<uint2*>(q + bq_pos(m, c, kp)) = make_uint2(ev, od);
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
        // gate_up 18.8 -> 16.9 us, the LM head 106.8 -> 81.7 us) where that
        // still leaves a block per CU (the qkv GEMM's 192 blocks of 32 rows
        // took longer than its 384 of 16: 2.488 -> 2.473 ms per M = 32 step)
        if (two_groups || (BT == 2 && (p.n + 31) / 32 >= 256)) launch_gemm_lds<2, 4, BT, 1280>(p, s);
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
