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
// 16 * acc exactly.  The B operand is the activation slice stored in LDS with
// the same per-8-column even/odd order, so A and B agree on the K order: a
// prologue kernel writes the int8 activations once into the workspace in
// that order, rows padded to whole 256-column slices with zeros, and each
// GEMM block copies its columns into LDS with global->LDS loads.
// K is split across blocks so that small row counts still fill the chip;
// split partial sums meet in an int32 workspace through atomic adds, and the
// last split to arrive at a row tile writes the epilogue and re-zeroes its
// part of the workspace (no waiting anywhere).
#include "hq_device.h"
#include "hq_internal.h"

namespace hq {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kTileRows = 64;     // 4 waves x 16 rows
constexpr int kSlice = 256;       // K columns staged per iteration
constexpr int kMaxBatch = 32;     // sequences per launch (two 16-wide B tiles)
constexpr int kMaxSlices = 10;    // K slices one block covers (its weights in flight at once)

struct GemmParams {
    const int8_t* x;          // [m, kp] de-interleaved per 8 columns, zero past K
    const float* act;         // [m]
    const uint8_t* w;         // [N, K/2]
    const float* ws;          // [N]
    float* out;               // [m, N]
    int32_t* acc_out;         // nullable [m, N]
    int32_t* acc;             // workspace [m, N] (zero between calls)
    int32_t* counters;        // workspace [tiles]
    int m, n, k, kp;          // kp: padded row stride of x (a multiple of kSlice)
    int slices_per_split;
    int splits;
};

// De-interleave 8 int8 columns (a, b = the two little-endian dwords) into
// [even columns | odd columns].
__device__ __forceinline__ void deinterleave8(uint32_t a, uint32_t b, uint32_t& ev, uint32_t& od)
{
    ev = (a & 0xFFu) | ((a >> 8) & 0xFF00u) | ((b & 0xFFu) << 16) | ((b & 0xFF0000u) << 8);
    od = ((a >> 8) & 0xFFu) | ((a >> 16) & 0xFF00u) | ((b & 0xFF00u) << 8) | (b & 0xFF000000u);
}

// A block covers one 64-row tile over a range of at most kMaxSlices K
// slices.  Every lane issues all of its weight loads for the range first
// (32 bytes of its row per slice), so a block keeps up to 64 KB of weights in
// flight; the activation columns of the range are staged in LDS (de-interleaved,
// once per block) while those loads travel, and the MFMAs then run from
// registers and LDS without further barriers.
template <int BT>
__global__ __launch_bounds__(kBlock) void gemm_mfma_kernel(GemmParams p)
{
    constexpr int MP = 16 * BT;                 // padded batch
    __shared__ __align__(16) uint8_t xs[MP * kSlice * kMaxSlices];
    __shared__ int last_flag;

    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid & (kWave - 1);
    const int tile = blockIdx.x;
    const int split = blockIdx.y;
    const int row0 = tile * kTileRows + wave * 16;
    const int arow = row0 + (lane & 15);        // A row of this lane
    const int kb = lane >> 4;                   // 0..3: 64-column quarter of a slice
    const bool arow_ok = arow < p.n;
    const int half = p.k >> 1;
    const uint8_t* wrow = p.w + size_t(arow_ok ? arow : 0) * size_t(half);
    const int nslices = (p.k + kSlice - 1) / kSlice;
    const int s_begin = split * p.slices_per_split;
    const int ns = min(nslices, s_begin + p.slices_per_split) - s_begin;   // 1 .. kMaxSlices

    // A: 32 packed bytes (64 columns) of row `arow` per lane and slice: the
    // four lanes of a row read its slice bytes [16kb, 16kb+16) (wa) and
    // [64+16kb, 64+16kb+16) (wb), so each load instruction reads 64
    // contiguous bytes of each of its 16 rows
    uint4 wa[kMaxSlices], wb[kMaxSlices];
#pragma unroll
    for (int j = 0; j < kMaxSlices; ++j) {
        wa[j] = make_uint4(0, 0, 0, 0);
        wb[j] = make_uint4(0, 0, 0, 0);
        const int ca = (s_begin + j) * kSlice + 32 * kb;        // first column of wa
        const int cb = ca + 128;                                 // first column of wb
        if (j < ns && arow_ok && ca < p.k) wa[j] = *reinterpret_cast<const uint4*>(wrow + (ca >> 1));
        if (j < ns && arow_ok && cb < p.k) wb[j] = *reinterpret_cast<const uint4*>(wrow + (cb >> 1));
    }

    // stage x[:, range] (already de-interleaved, zero past K and in rows
    // m .. MP-1 of the workspace) into LDS, rows of ns*kSlice bytes
    const int rowb = ns * kSlice;
    const int chunks = MP * rowb / 16;
    const int k0 = s_begin * kSlice;
    const uint32_t xs0 = lds_addr(xs);
    for (int q0 = wave * kWave; q0 < chunks; q0 += kBlock) {
        const int q = q0 + lane;
        const int mm = q / (rowb / 16);
        const int c = (q % (rowb / 16)) * 16;
        if (q < chunks) dma16(p.x, uint32_t(mm * p.kp + k0 + c), xs0 + uint32_t(q0) * 16u);
    }
    wait_all_memory();
    __syncthreads();

    i32x4 acc[BT];
#pragma unroll
    for (int b = 0; b < BT; ++b) acc[b] = i32x4{0, 0, 0, 0};
#pragma unroll
    for (int sl = 0; sl < kMaxSlices; ++sl) {
        if (sl < ns) {
            const uint32_t wd[8] = {wa[sl].x, wa[sl].y, wa[sl].z, wa[sl].w, wb[sl].x, wb[sl].y, wb[sl].z, wb[sl].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t m4 = 0xF0F0F0F0u;
                const i32x4 a = {int((wd[2 * j] << 4) & m4), int(wd[2 * j] & m4),
                                 int((wd[2 * j + 1] << 4) & m4), int(wd[2 * j + 1] & m4)};
                // columns of chunk j: wa holds [32kb, 32kb+32), wb [128+32kb, 128+32kb+32)
                const int cofs = sl * kSlice + (j >> 1) * 128 + 32 * kb + 16 * (j & 1);
#pragma unroll
                for (int b = 0; b < BT; ++b) {
                    const uint4 xv = *reinterpret_cast<const uint4*>(xs + (16 * b + (lane & 15)) * rowb + cofs);
                    const i32x4 bv = {int(xv.x), int(xv.y), int(xv.z), int(xv.w)};
                    acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bv, acc[b], 0, 0, 0);
                }
            }
        }
    }

    // D layout: lane holds rows 4*(lane/16) + r, column lane % 16.
    const int col_m = lane & 15;
    const int rbase = row0 + 4 * (lane >> 4);
    if (p.splits == 1) {
#pragma unroll
        for (int b = 0; b < BT; ++b) {
            const int mm = 16 * b + col_m;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int n = rbase + r;
                if (mm < p.m && n < p.n) {
                    const int a = acc[b][r] >> 4;
                    p.out[size_t(mm) * p.n + n] = (float(a) * p.act[mm]) * p.ws[n];
                    if (p.acc_out) p.acc_out[size_t(mm) * p.n + n] = a;
                }
            }
        }
        return;
    }
#pragma unroll
    for (int b = 0; b < BT; ++b) {
        const int mm = 16 * b + col_m;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int n = rbase + r;
            if (mm < p.m && n < p.n) atomicAdd(p.acc + size_t(mm) * p.n + n, acc[b][r] >> 4);
        }
    }
    wait_all_memory();   // this thread's atomic adds have been performed
    __syncthreads();
    if (tid == 0) {
        const int ticket = atomicAdd(p.counters + tile, 1);
        last_flag = (ticket == p.splits - 1);
    }
    __syncthreads();
    if (!last_flag) return;
    const int trows = min(kTileRows, p.n - tile * kTileRows);
    for (int e = tid; e < p.m * trows; e += kBlock) {
        const int mm = e / trows;
        const int n = tile * kTileRows + e % trows;
        int32_t* cell = p.acc + size_t(mm) * p.n + n;
        const int a = read_i(cell);
        p.out[size_t(mm) * p.n + n] = (float(a) * p.act[mm]) * p.ws[n];
        if (p.acc_out) p.acc_out[size_t(mm) * p.n + n] = a;
        publish_i(cell, 0);
    }
    if (tid == 0) publish_i(p.counters + tile, 0);
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
    size_t acc_off, counter_off, q_off, act_off, total;
};

static size_t al256(size_t v) { return (v + 255) & ~size_t(255); }

static int padded_k(int k) { return (k + kSlice - 1) / kSlice * kSlice; }
static int padded_m(int m) { return (m + kMaxBatch - 1) / kMaxBatch * kMaxBatch; }

static GemmLayout gemm_layout(int m, int n, int k)
{
    const int mb = m < kMaxBatch ? m : kMaxBatch;
    GemmLayout L{};
    L.acc_off = 0;
    L.counter_off = al256(size_t(mb) * size_t(n) * 4);
    L.q_off = L.counter_off + al256(size_t((n + kTileRows - 1) / kTileRows) * 4);
    // de-interleaved activations, padded_m(m) rows of padded_k(k) bytes;
    // padding bytes are never written (zero from the initial fill)
    L.act_off = L.q_off + al256(size_t(padded_m(m)) * size_t(padded_k(k)));
    L.total = L.act_off + al256(size_t(m) * 4);
    return L;
}

// x: the de-interleaved padded activations in the workspace.
static hipError_t run_gemm(const int8_t* x, const float* act, const uint8_t* w, const float* ws,
                           float* out, int m, int n, int k, int32_t* acc_out, char* workspace,
                           hipStream_t s)
{
    const GemmLayout L = gemm_layout(m, n, k);
    const int kp = padded_k(k);
    const int tiles = (n + kTileRows - 1) / kTileRows;
    const int nslices = (k + kSlice - 1) / kSlice;
    // about one block per CU, each covering at most kMaxSlices slices; a
    // split K costs a round of atomic adds and a ticket, so shapes with
    // enough row tiles to fill half the chip are not split
    int want = tiles >= 128 ? 1 : (256 + tiles - 1) / tiles;
    if (want < 1) want = 1;
    if (want > nslices) want = nslices;
    int per = (nslices + want - 1) / want;
    if (per > kMaxSlices) per = kMaxSlices;
    const int splits = (nslices + per - 1) / per;
    for (int m0 = 0; m0 < m; m0 += kMaxBatch) {
        GemmParams p{};
        p.m = m - m0 < kMaxBatch ? m - m0 : kMaxBatch;
        p.x = x + size_t(m0) * kp;
        p.act = act + m0;
        p.w = w; p.ws = ws;
        p.out = out + size_t(m0) * n;
        p.acc_out = acc_out ? acc_out + size_t(m0) * n : nullptr;
        p.acc = reinterpret_cast<int32_t*>(workspace + L.acc_off);
        p.counters = reinterpret_cast<int32_t*>(workspace + L.counter_off);
        p.n = n; p.k = k; p.kp = kp;
        p.slices_per_split = per;
        p.splits = splits;
        if (p.m <= 16)
            hipLaunchKernelGGL(gemm_mfma_kernel<1>, dim3(tiles, splits), dim3(kBlock), 0, s, p);
        else
            hipLaunchKernelGGL(gemm_mfma_kernel<2>, dim3(tiles, splits), dim3(kBlock), 0, s, p);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int gemm_padded_k(int k) { return padded_k(k); }
int gemm_padded_m(int m) { return padded_m(m); }
size_t gemm_scratch_bytes(int m, int n, int k) { return gemm_layout(m, n, k).q_off; }
hipError_t gemm_run(const int8_t* x, const float* act, const uint8_t* w, const float* ws, float* out, int m, int n,
                    int k, char* scratch, hipStream_t s)
{
    return run_gemm(x, act, w, ws, out, m, n, k, nullptr, scratch, s);
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
    const hipError_t e = run_gemm(q, act_scales, weights, scales, output, m, rows, width, acc_out, ws, s);
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
    const hipError_t e = run_gemm(q, act, weights, scales, output, m, rows, width, acc_out, ws, s);
    return e == hipSuccess ? HQ_OK : HQ_ERR_LAUNCH;
}
