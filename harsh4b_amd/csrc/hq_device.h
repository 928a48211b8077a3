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

#include <utility>

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
// Halving trees: at level o, partial i is paired with partial i + o.  Within
// a 16-lane row the levels use DPP row_shl (lane i reads lane i + o); across
// rows gfx950's v_permlane16_swap / v_permlane32_swap pair lane i with lane
// i + 16 / i + 32.  Every level is one VALU op, no LDS round trip, and the
// pairing is exactly the oracle's tree_sum order (fp32 addition is
// commutative, so which lane of a pair adds is irrelevant).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0u, __builtin_bit_cast(unsigned, v),
                                                                  CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int kRowShl1 = 0x101, kRowShl2 = 0x102, kRowShl4 = 0x104, kRowShl8 = 0x108;

// Cross-row exchanges.  v_permlane32_swap(x, y) swaps the upper 32 lanes of
// x with the lower 32 lanes of y (v_permlane16_swap: odd 16-lane rows of x
// with even rows of y); both registers are read and written, so the
// instructions are written as inline asm with two in/out operands (the
// compiler's builtin for them folds one of the two results away); the
// s_nop wait states on either side cover the VALU-write -> swap-read and
// swap-write -> VALU-read hazards the compiler cannot see through asm.  With
// y = 0 on entry, lane i < 32 ends with x = v[i], y = v[i + 32]
// (v[i + 16] for the 16-lane form, lanes i < 16 of each 32-lane half).
__device__ __forceinline__ void swap32(unsigned& x, unsigned& y)
{
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(x), "+v"(y));
}
__device__ __forceinline__ void swap16(unsigned& x, unsigned& y)
{
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(x), "+v"(y));
}

// Levels 32 and 16 of a 64-lane tree, valid in lanes 0..15.
__device__ __forceinline__ float levels_32_16(float v)
{
    unsigned x = __builtin_bit_cast(unsigned, v), y = 0u;
    swap32(x, y);
    v = __builtin_bit_cast(float, x) + __builtin_bit_cast(float, y);
    x = __builtin_bit_cast(unsigned, v);
    y = 0u;
    swap16(x, y);
    return __builtin_bit_cast(float, x) + __builtin_bit_cast(float, y);
}

// 16-lane tree within each DPP row; the total is valid in lane 0 of the row.
__device__ __forceinline__ float row_tree_sum16(float v)
{
    v = v + dpp_f<kRowShl8>(v);
    v = v + dpp_f<kRowShl4>(v);
    v = v + dpp_f<kRowShl2>(v);
    v = v + dpp_f<kRowShl1>(v);
    return v;
}

// 64-lane tree; the total is valid in lane 0.
__device__ __forceinline__ float wave_tree_sum64(float v) { return row_tree_sum16(levels_32_16(v)); }

// 64-lane tree, total broadcast to every lane.
__device__ __forceinline__ float wave_tree_sum64_all(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                         __builtin_bit_cast(unsigned, wave_tree_sum64(v)), 0));
}

// Integer sum over aligned groups of 8 lanes; valid in the group's first lane.
__device__ __forceinline__ int group8_isum(int v)
{
    v += dpp_i<kRowShl4>(v);
    v += dpp_i<kRowShl2>(v);
    v += dpp_i<kRowShl1>(v);
    return v;
}

// Integer sum over the wave (order-free); valid in lane 0.
__device__ __forceinline__ int wave_isum64(int v)
{
    unsigned x = unsigned(v), y = 0u;
    swap32(x, y);
    x = unsigned(int(x) + int(y));
    y = 0u;
    swap16(x, y);
    v = int(x) + int(y);
    v += dpp_i<kRowShl8>(v);
    return group8_isum(v);
}

// Max over the wave (order-free), read from lane 0 and broadcast to every lane.
__device__ __forceinline__ float wave_max64_all(float v)
{
    unsigned x = __builtin_bit_cast(unsigned, v), y = x;
    swap32(x, y);
    v = fmaxf(__builtin_bit_cast(float, x), __builtin_bit_cast(float, y));
    x = __builtin_bit_cast(unsigned, v);
    y = x;
    swap16(x, y);
    v = fmaxf(__builtin_bit_cast(float, x), __builtin_bit_cast(float, y));
    v = fmaxf(v, dpp_f<kRowShl8>(v));
    v = fmaxf(v, dpp_f<kRowShl4>(v));
    v = fmaxf(v, dpp_f<kRowShl2>(v));
    v = fmaxf(v, dpp_f<kRowShl1>(v));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(unsigned, v), 0));
}

// Block barrier for LDS data only: the wave's LDS operations complete, then
// s_barrier.  Unlike __syncthreads it does not wait for the wave's global
// loads and stores, so weight loads issued before a block reduction keep
// streaming through it.
__device__ __forceinline__ void lds_sync()
{
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Block-wide (256 threads) max of non-negative values; `red` is 4 floats of LDS.
__device__ __forceinline__ float block_max_nonneg(float v, float* red)
{
    v = wave_max64_all(v);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = v;
    lds_sync();
    const float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    lds_sync();   // red may be written again after the return
    return r;
}

// Block-wide sum of 256 per-thread partials with the spec's halving tree
// (partial i + partial i+o for o = 128, 64, ..., 1).  `red` is 256 floats of
// LDS.  Every wave reads levels 128 and 64 of its lanes from LDS and runs
// the wave tree over the remaining 64, so every thread returns the total
// after one barrier.
__device__ __forceinline__ float block_tree_sum256(float v, float* red)
{
    const int t = threadIdx.x;
    red[t] = v;
    lds_sync();
    const int l = t & (kWave - 1);
    const float r = wave_tree_sum64_all((red[l] + red[l + 128]) + (red[l + 64] + red[l + 192]));
    lds_sync();   // red may be written again after the return
    return r;
}

// ---- cross-block hand-off without fences ------------------------------------
// A full fence (__threadfence) writes back the XCD's L2 and costs tens of
// microseconds when hundreds of blocks issue it, and same-address atomics
// serialise at ~20 ns each.  Blocks therefore publish data with agent-scope
// atomic stores (written through to the coherence point), wait for them to
// complete, and only then take a ticket; readers use agent-scope atomic
// loads.  publish_f/i, read_f/i are those accesses.
__device__ __forceinline__ void publish_f(float* p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish_i(int* p, int v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float read_f(const float* p)
{
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int read_i(const int* p)
{
    return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until every memory operation this thread issued has completed.
__device__ __forceinline__ void wait_all_memory() { __builtin_amdgcn_s_waitcnt(0); }
// Wait until at most n (0..2) of this wave's vector memory loads are
// outstanding (they complete in issue order); n is wave-uniform.
__device__ __forceinline__ void wait_vm_le(int n)
{
    if (n >= 2) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    else if (n == 1) asm volatile("s_waitcnt vmcnt(1)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// A pointer every lane holds the same value of, as a scalar (SGPR) value:
// loads through it take a 32-bit per-lane offset.
template <class T>
__device__ __forceinline__ const T* uniform_ptr(const T* p)
{
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(v >> 32));
    return reinterpret_cast<const T*>((uint64_t(hi) << 32) | lo);
}

// A raw buffer resource over [p, p + bytes) (gfx9 layout, stride 0): loads
// through it take a 32-bit lane offset plus a scalar offset, so a burst of
// loads at scalar distances from one lane address holds one VGPR of
// address; a load at or past `bytes` returns 0 and touches no memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* p, int bytes = 0x7fffffff)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(uniform_ptr(p)), 0,
                                             __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}
// Cache-policy bit of a buffer access that is coherent at agent scope (the
// bits of an agent-scope atomic load or store).
constexpr int kAgentSC1 = 16;

// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void* p)
{
    return uint32_t(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}

// One 16-byte global->LDS copy per active lane (gfx950 global_load_lds_dwordx4):
// lane i reads base + off (base the same in every lane) and writes LDS bytes
// lds + 16*i .. +15 (lds the same in every lane).  Written as asm (the
// compiler's own tracking of this instruction would make unrelated later
// instructions wait for it); the data may be read once the wave's memory
// operations have been waited for (wait_all_memory) and, for other waves,
// after a barrier.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds)
{
    const uint32_t m = __builtin_amdgcn_readfirstlane(lds);
    const void* ub = uniform_ptr(base);
    uint32_t saved;   // m0 is reserved to the compiler: restore it
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
                 "global_load_lds_dwordx4 %2, %3\n\ts_nop 0\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(m), "v"(off), "s"(ub)
                 : "memory");
}

constexpr int kTicketGroup = 32;   // blocks per first-level ticket counter

// Two-level arrival ticket for `nblocks` blocks, called by one thread per
// block after __syncthreads() has ordered the block's published writes.
// counters: [ceil(nblocks / 32) group counters][1 top counter], zero between
// uses; the function leaves them zero again.  Returns true in exactly one
// block, the last to arrive, after all others have published.
__device__ __forceinline__ bool last_block_ticket(int* counters, int block, int nblocks)
{
    const int groups = (nblocks + kTicketGroup - 1) / kTicketGroup;
    const int g = block / kTicketGroup;
    const int gsize = min(kTicketGroup, nblocks - g * kTicketGroup);
    if (atomicAdd(counters + g, 1) != gsize - 1) return false;
    publish_i(counters + g, 0);
    if (atomicAdd(counters + groups, 1) != groups - 1) return false;
    publish_i(counters + groups, 0);
    return true;
}
__host__ __device__ constexpr int ticket_words(int nblocks)
{
    return (nblocks + kTicketGroup - 1) / kTicketGroup + 1;
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
// Byte position of de-interleaved column byte c (c = xq_offset(column)) of
// row `row` in a batched GEMM input of row stride kp: the rows go in tiles
// of 16 (tile t spans bytes [16 t kp, 16 (t + 1) kp), as 16 rows of kp
// would), and within a tile every double step of 128 columns is two 1 KB
// blocks, block h holding bytes 32 q + 16 h .. + 15 of the step for rows
// r = 0..15 at (16 q + r) * 16 -- the order in which the 64 lanes of an
// MFMA B operand (lane 16 q + r: row r, bytes 32 q + 16 h of the step) load
// them, so each wave load of the operand reads 1 KB of contiguous memory
// instead of a half of 16 rows' cache lines.
__device__ __forceinline__ size_t bq_pos(int row, int c, int kp)
{
    return size_t(row >> 4) * 16 * size_t(kp) + size_t(c >> 7) * 2048 + size_t((c >> 4) & 1) * 1024 +
           size_t((c >> 5) & 3) * 256 + size_t(row & 15) * 16 + size_t(c & 15);
}

__device__ __forceinline__ int8_t quant_i8(float v, float inv)
{
    float q = __builtin_rintf(v * inv);
    q = fminf(fmaxf(q, -127.0f), 127.0f);
    return static_cast<int8_t>(static_cast<int>(q));
}

// ---- {value, epoch} entries of the batched step's launch tails -------------------
//
// A launch's blocks hand values to its last blocks as 64-bit entries, the
// value's bits in the low word and the launch's epoch in the high word,
// with agent-scope stores and loads (no fences).  The epoch is
// (step << 8) | launch id, the step counter running 1 .. kEpochSteps - 1:
// the step's first kernel clears every entry (epoch 0) when the counter
// wraps, so an entry's epoch equals the launch's only when the launch itself
// wrote it, however long the workspace lives.
constexpr uint32_t kEpochSteps = 1u << 23;

__device__ __forceinline__ bool tail_ready(uint64_t v, uint32_t ep)
{
    return uint32_t(v >> 32) == ep;
}
__device__ __forceinline__ uint64_t tail_load(const uint64_t* p)
{
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void tail_store(uint64_t* p, float v, uint32_t ep)
{
    __hip_atomic_store(p, (uint64_t(ep) << 32) | uint64_t(f32_bits(v)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
constexpr unsigned kTailSpinLimit = 1u << 22;   // rounds a tail waits before it gives up (HQ_STEP_SYNC)

// f(0) .. f(N-1) with compile-time indices (register arrays stay in registers)
template <class F, int... J>
__device__ __forceinline__ void unrolled_impl(F&& f, std::integer_sequence<int, J...>)
{
    (f(std::integral_constant<int, J>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void unrolled(F&& f)
{
    unrolled_impl(f, std::make_integer_sequence<int, N>{});
}

}  // namespace hq
