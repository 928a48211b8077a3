// hq_int4.h - building blocks of the packed-int4 x int8 dot products shared
// by the GEMV kernels and the fused layer kernel (gfx950).
//
// Weights: two's-complement nibbles, low nibble = even column, 16 bytes (32
// values) per chunk.  Activations: int8 in LDS, de-interleaved per 8 columns
// (xq_offset), so one weight dword meets one activation dword per nibble
// half: for a weight dword w, (w << 4) & 0xF0F0F0F0 holds 16*low nibbles and
// w & 0xF0F0F0F0 holds 16*high nibbles as signed bytes, and v_dot4_i32_i8
// gives 16 * sum(w*x) exactly.
#pragma once

#include "hq_device.h"

namespace hq {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Weights are read exactly once per step: stream them past the caches.
// The pointer is global memory: a global (not flat) load waits on the
// vector-memory counter only, never on the LDS counter.
__device__ __forceinline__ uint4 load_w16(const uint8_t* p)
{
    const u32x4 v = __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 16 * sum(w * x) over one 16-byte weight chunk, accumulated into two
// independent integer chains (integer addition is exact in any order).
__device__ __forceinline__ void dot_chunk(uint4 w, const uint8_t* xs_chunk, int& a0, int& a1)
{
    const uint4 xa = *reinterpret_cast<const uint4*>(xs_chunk);
    const uint4 xb = *reinterpret_cast<const uint4*>(xs_chunk + 16);
    const int m = int(0xF0F0F0F0u);
    a0 = __builtin_amdgcn_sdot4(int(w.x << 4) & m, int(xa.x), a0, false);
    a1 = __builtin_amdgcn_sdot4(int(w.x) & m, int(xa.y), a1, false);
    a0 = __builtin_amdgcn_sdot4(int(w.y << 4) & m, int(xa.z), a0, false);
    a1 = __builtin_amdgcn_sdot4(int(w.y) & m, int(xa.w), a1, false);
    a0 = __builtin_amdgcn_sdot4(int(w.z << 4) & m, int(xb.x), a0, false);
    a1 = __builtin_amdgcn_sdot4(int(w.z) & m, int(xb.y), a1, false);
    a0 = __builtin_amdgcn_sdot4(int(w.w << 4) & m, int(xb.z), a0, false);
    a1 = __builtin_amdgcn_sdot4(int(w.w) & m, int(xb.w), a1, false);
}

// Row sums of a wave whose rows are read by LPR lanes each (RPW = 64/LPR
// rows): returns the integer total of row r (wave-uniform).  Integer sums
// are exact in any order.
template <int LPR>
__device__ __forceinline__ int row_isum(int v, int r)
{
    // v: per-lane partial; returns the total of row r of the wave (uniform)
    if constexpr (LPR == 8) {
        v = group8_isum(v);
        return __builtin_amdgcn_readlane(v, 8 * r);
    } else {
        v += dpp_i<kRowShl8>(v);
        v = group8_isum(v);
        if constexpr (LPR == 16) return __builtin_amdgcn_readlane(v, 16 * r);
        if constexpr (LPR == 32)
            return __builtin_amdgcn_readlane(v, 32 * r) + __builtin_amdgcn_readlane(v, 32 * r + 16);
        return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) +
               __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48);
    }
}

}  // namespace hq
