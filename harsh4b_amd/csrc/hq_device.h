// hq_device.h - device-side building blocks shared by the hq kernels (gfx950).
//
// Numeric spec v1: every floating-point step below is one IEEE fp32
// operation (the library is compiled with -ffp-contract=off, so a*b+c is two
// roundings unless written as fmaf).  Division and sqrt are the correctly
// rounded HIP defaults.  Reductions whose order changes fp32 bits use the
// fixed trees named in each helper; integer and max reductions are
// order-free.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hq {

constexpr int kBlock = 256;   // threads per block for every hq kernel
constexpr int kWave = 64;

__device__ __forceinline__ float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }

// 2^k for k in [-126, 127].
__device__ __forceinline__ float pow2i(int k) { return bits_f32(uint32_t(k + 127) << 23); }

// exp(x): Cody & Waite reduction (n = rint(x*log2 e), r = x - n*ln2 with a
// two-part ln2 through fmaf), degree-7 Taylor polynomial of e^r in Horner
// form, scaling by 2^n as two exact power-of-two multiplies.  x < -87 gives
// exactly 0 (never a subnormal), x > 88.72284 gives +inf.
__device__ __forceinline__ float spec_expf(float x)
{
    if (x != x) return x;
    if (x > 0x1.62e430p+6f) return __builtin_inff();
    if (x < -87.0f) return 0.0f;
    const float n = __builtin_rintf(x * 0x1.715476p+0f);
    float r = __builtin_fmaf(-n, 0x1.62e400p-1f, x);
    r = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int ni = int(n);
    const int n1 = ni / 2;
    const int n2 = ni - n1;
    p = p * pow2i(n1);
    p = p * pow2i(n2);
    return p;
}

// fp16 storage (RNE on the way in, exact widening on the way out).
__device__ __forceinline__ uint16_t f32_to_f16(float x)
{
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}
__device__ __forceinline__ float f16_to_f32(uint16_t h)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// ---- wave-level reductions -------------------------------------------------
// Halving tree across `width` lanes (width a power of two <= 64): after the
// xor steps width/2 ... 1 every lane of the group holds the tree in which
// partial i is paired with i + o at each level o -- the order the oracle's
// tree_sum uses.  fp32 addition is commutative, so lane i and lane i^o form
// the same sum.
template <int WIDTH>
__device__ __forceinline__ float tree_sum(float v)
{
#pragma unroll
    for (int o = WIDTH / 2; o >= 1; o >>= 1) v = v + __shfl_xor(v, o, kWave);
    return v;
}

template <int WIDTH>
__device__ __forceinline__ int isum(int v)
{
#pragma unroll
    for (int o = WIDTH / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

template <int WIDTH>
__device__ __forceinline__ float fmax_group(float v)
{
#pragma unroll
    for (int o = WIDTH / 2; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// Block-wide (256 threads) max of non-negative values; `red` is 4 floats of LDS.
__device__ __forceinline__ float block_max_nonneg(float v, float* red)
{
    v = fmax_group<kWave>(v);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = v;
    __syncthreads();
    const float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    return r;
}

// Block-wide sum of 256 per-thread partials with the spec's halving tree
// (partial i + partial i+o for o = 128, 64, ..., 1).  `red` is 256 floats of
// LDS.  Levels 128 and 64 go through LDS, the last 64 lanes through the
// wave tree.  Every thread returns the total.
__device__ __forceinline__ float block_tree_sum256(float v, float* red)
{
    const int t = threadIdx.x;
    red[t] = v;
    __syncthreads();
    if (t < 128) red[t] = red[t] + red[t + 128];
    __syncthreads();
    float r = 0.0f;
    if (t < 64) {
        r = red[t] + red[t + 64];
        r = tree_sum<kWave>(r);
        if (t == 0) red[0] = r;
    }
    __syncthreads();
    r = red[0];
    __syncthreads();
    return r;
}

// Argmax order of np.argmax: a NaN beats any number, the lowest index wins
// among equals (and among NaNs).  Returns true when (a, ia) is preferred.
__device__ __forceinline__ bool argmax_better(float a, int ia, float b, int ib)
{
    const bool an = a != a, bn = b != b;
    if (an != bn) return an;
    if (an) return ia < ib;
    if (a != b) return a > b;
    return ia < ib;
}

// LDS byte offset of activation element i in the de-interleaved int8 layout
// the GEMV reads: each group of 8 columns is stored as the 4 even columns
// followed by the 4 odd columns.
__device__ __forceinline__ int xq_offset(int i)
{
    return (i & ~7) + ((i & 1) << 2) + ((i & 7) >> 1);
}

// Symmetric int8 quantization of one value with inv = 127 / amax.
__device__ __forceinline__ int8_t quant_i8(float v, float inv)
{
    float q = __builtin_rintf(v * inv);
    q = fminf(fmaxf(q, -127.0f), 127.0f);
    return static_cast<int8_t>(static_cast<int>(q));
}

}  // namespace hq
