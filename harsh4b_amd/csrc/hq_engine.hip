// hq_engine.hip - every decoder layer of one decode step in a single
// persistent kernel (gfx950).
//
// The per-layer sequence is the one of LiteSparkQwen.forward_token
// (cpu_lightspark.py:431-459 in the reference repository), as five phases:
//   P1  RMSNorm(input) -> int8 quant -> fused qkv GEMV
//   P2  qk-norm -> RoPE -> fp16 KV append -> GQA attention
//   P3  int8 quant -> o GEMV -> residual add
//   P4  RMSNorm(post) -> int8 quant -> fused gate_up GEMV -> SwiGLU
//   P5  int8 quant -> down GEMV -> residual add
// with exactly the numerics of the per-kernel path (hq_gemv.hip,
// hq_attention.hip): the same reduction trees, the same exp, the same
// operation order, so both paths give the same bits.
//
// Why one kernel.  At batch 1 a GEMV of 5-25 MB is too short to reach HBM
// bandwidth on its own: every kernel boundary drains the memory pipeline
// and the next kernel starts its weight stream only after its launch.  Here
// one block per CU (1024 threads) lives for the whole step, and the weights
// of each GEMV are loaded into registers about two phases before they are
// used, so the HBM stream runs through the phase boundaries.
//
// Phase hand-off without fences or barriers.  Each phase's output vector is
// published as 64-bit entries {fp32 value, 32-bit epoch} with agent-scope
// atomic stores (written through to the coherence point, single-copy atomic),
// and consumers poll the entries they need with agent-scope atomic loads
// until every epoch is current.  Epochs grow by 5 per layer from a counter
// kept in the workspace, so no buffer needs clearing between steps.
//
// Wave roles.  Vector-memory operations of one wave complete in issue order,
// so a poll issued behind a weight prefetch would wait for the prefetch.
// Waves 0-3 ("input waves") therefore never load weights: they load norm
// weights, poll phase inputs, load KV-cache chunks and publish attention
// partials.  Waves 4-15 ("weight waves") hold the weight prefetch and do the
// GEMV dot products; they poll only where their prefetch has landed by then
// (P1, P5).  Barriers are block-wide and every thread executes each of them,
// so role-specific work is predicated, never a divergent barrier.
//
// Every wait is bounded: a thread that polls kPollBudget times gives up,
// raises HQ_STEP_SYNC in the status word and never waits again, so the
// kernel always finishes.  The grid (at most one block per CU, fewer blocks
// than CUs) is co-resident by construction.
#include "hq_device.h"
#include "hq_int4.h"
#include "hq_internal.h"

namespace hq {
namespace eng {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / kWave;         // 16
constexpr int kIThreads = 256;                   // waves 0-3
constexpr int kD = 128;                          // head_dim
constexpr int kG = 4;                            // query heads per kv head (max)
constexpr int kCPB = 4;                          // attention chunks per work item
constexpr int kRow = kD + 8;                     // padded LDS row of a K/V chunk
constexpr int kMaxVec = 10240;                   // largest phase input (floats)
constexpr int kMaxHidden = 2560;
constexpr int kMaxOwn = 16;                      // residual rows per block
constexpr int kMaxRes = 48;                      // outputs of one GEMV phase per block
constexpr int kMaxLayers = 64;                   // layer table copy in LDS
constexpr int kWaveStage = 10 * 1024;            // stage bytes per weight wave (10 chunk slots)
constexpr unsigned kPollBudget = 1u << 17;

// Weight-wave layouts: LPR lanes per row, MAXC 16-byte chunks per lane.
constexpr int kQkvLPR = 32, kQkvMAXC = 3;        // K <= 3072, 24 rows per block
constexpr int kOLPR = 64, kOMAXC = 2;            // K <= 4096, 12 rows
constexpr int kGuLPR = 8, kGuHalf = 5;           // K <= 2560 (2 x 5 chunks), 48 gate/up pairs
constexpr int kDownLPR = 64, kDownMAXC = 5;      // K <= 10240, 12 rows
constexpr int kWWaves = kWaves - kIThreads / kWave;   // 12
// Phase inputs held in registers: hidden vectors by the input threads (256),
// the attention output by the input threads, the SwiGLU output by all.
constexpr int kHidNPT = kMaxHidden / kIThreads;       // 10
constexpr int kAttNPT = 16;                           // heads*D <= 4096
constexpr int kActNPT = kMaxVec / kThreads;           // 10

}  // namespace eng

struct EngineParams {
    const hq_layer* layers;   // device table [L]
    int L, H, I, heads, kv_heads, G, qkv_rows;
    float eps;
    const float* rope_cos;
    const float* rope_sin;
    uint16_t* keys;
    uint16_t* values;
    long long kv_layer;       // cache elements per layer
    int kv_stride;            // cache elements per position
    int capacity;
    const int32_t* position;
    int32_t* status;
    float* x;                 // residual stream: embedding in, final out
    uint64_t* ll_x3;          // [H] x after o + residual
    uint64_t* ll_x5;          // [H] x after down + residual
    uint64_t* ll_qkv;         // [qkv_rows]
    uint64_t* ll_att;         // [heads * D]
    uint64_t* ll_act;         // [I]
    uint32_t* epoch;
    float* part;              // attention split partials
    int32_t* counters;        // [kv_heads] split tickets
    int max_chunks;
    uint32_t* trace;          // HQ_ENGINE_TRACE builds: phase timestamps
};

// Phase timestamps (builds with -DHQ_ENGINE_TRACE only): the low 32 bits of
// the 100 MHz wall clock at fixed points of layers kTraceL0 .. kTraceL0+3,
// from lane 0 of every wave, kept in LDS (a global store would join the
// wave's vector-memory queue and shift the waits being measured) and copied
// at the end to trace[((block*4 + layer-kTraceL0)*16 + point)*16 + wave]; the
// attention's own points follow for blocks gridDim.x + block.
#ifdef HQ_ENGINE_TRACE
constexpr int kTraceL0 = 16;
#define ENG_MARK(point)                                                                          \
    do {                                                                                         \
        const int t_ = opaque_tid();                                                             \
        if ((t_ & (kWave - 1)) == 0 && l >= kTraceL0 && l < kTraceL0 + 4)                        \
            trace_s[((l - kTraceL0) * 16 + (point)) * 16 + t_ / kWave] = uint32_t(wall_clock64()); \
    } while (0)
// sub-phase points: mk points at the 16x16 block of the layer (or nullptr)
#define SUB_MARK(mk, point)                                                                      \
    do {                                                                                         \
        const int t_ = opaque_tid();                                                             \
        if ((mk) != nullptr && (t_ & (kWave - 1)) == 0)                                          \
            (mk)[(point) * 16 + t_ / kWave] = uint32_t(wall_clock64());                          \
    } while (0)
#else
#define ENG_MARK(point) do { } while (0)
#define SUB_MARK(mk, point) do { (void)(mk); } while (0)
#endif

namespace {

using namespace eng;

__device__ __forceinline__ void ll_store(uint64_t* p, float v, uint32_t epoch)
{
    __hip_atomic_store(p, (uint64_t(epoch) << 32) | uint64_t(f32_bits(v)), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ll_load(const uint64_t* p)
{
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool ll_ready(uint64_t v, uint32_t epoch)
{
    return int32_t(uint32_t(v >> 32) - epoch) >= 0;
}

__device__ __forceinline__ int split_begin(int n, int b, int nb);


__device__ __forceinline__ int split_begin(int n, int b, int nb)
{
    return int((long long)n * b / nb);
}

// The thread index, opaque to the optimizer.  Addresses derived from it
// inside the layer loop are loop-invariant, and hoisting all of them out of
// the loop would hold more registers than the loop body itself needs.
__device__ __forceinline__ int opaque_tid()
{
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

__device__ __forceinline__ int lane_id() { return opaque_tid() & (kWave - 1); }

// The input waves publish a phase's outputs res[0, n) to dst[0, n).  Weight
// waves issue no global stores: on gfx9 a store's data registers are read
// after issue, and the compiler's wait before reusing them would, behind the
// weight wave's untracked prefetch loads (dma16), wait for those as well.
__device__ __forceinline__ void publish_rows(const float* res, uint64_t* dst, int n, uint32_t epoch)
{
    const int t = opaque_tid();
    if (t < kIThreads)
        for (int i = t; i < n; i += kIThreads) ll_store(dst + i, res[i], epoch);
}

// Block barrier for this kernel: the wave's LDS operations complete, then
// s_barrier.  __syncthreads() also carries a workgroup release fence, which
// waits for the wave's outstanding global->LDS weight loads (they are LDS
// writes) and would make every barrier wait for the weight prefetch.  No
// LDS data handed between waves here comes from those loads: a weight wave
// reads only its own staged weights, after waiting for them itself.  The
// memory clobber keeps the compiler from moving memory accesses across.
__device__ __forceinline__ void block_sync()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Pointers read from the device layer table are generic to the compiler;
// reading through a global-address-space pointer gives global (not flat)
// loads, which wait on the vector-memory counter only.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gmem(const T* p)
{
    return (const __attribute__((address_space(1))) T*)p;
}

// A pointer every lane holds the same value of, as a scalar (SGPR) value.
template <class T>
__device__ __forceinline__ const T* uniform_ptr(const T* p)
{
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(v >> 32));
    return reinterpret_cast<const T*>((uint64_t(hi) << 32) | lo);
}


// Wave 0 of the block waits until 64 entries spread evenly over src[0, n)
// are current (lane i watches entry (i+1)*n/64 - 1); the block then reads
// the whole vector in one burst (poll_into) after a barrier.  Spinning with
// one wave instead of the readers of all n entries keeps the fabric quiet
// while the producers' stores travel: a single watching wave on spread
// entries made a 2560-entry hand-off between 256 blocks 1.0 us shorter than
// every reader spinning on its own entries.
__device__ __forceinline__ void watch_spread(const uint64_t* src, int n, uint32_t epoch, unsigned& budget,
                                             int32_t* status)
{
    const int t = opaque_tid();
    if (t < kWave) {
        const int e = ((t + 1) * n) / kWave - 1;
        if (e >= 0) {
            uint64_t w = ll_load(src + e);
            while (!ll_ready(w, epoch) && budget != 0) {
                __builtin_amdgcn_s_sleep(1);
                if (--budget == 0) atomicOr(status, HQ_STEP_SYNC);
                w = ll_load(src + e);
            }
        }
    }
}

// Polls entries t, t+T, ... of src[0, n) (threads t < T) until their epoch
// is current and returns their values in out[] (0 past n).
template <int T, int NPT>
__device__ __forceinline__ void poll_into(const uint64_t* src, int n, uint32_t epoch, float (&out)[NPT],
                                          unsigned& budget, int32_t* status)
{
    const int t = opaque_tid();
    // entries past n are not loaded and count as current; the others are at
    // src + t + T*j, affine in t (one offset register for all j)
    const uint64_t done = uint64_t(epoch) << 32;
    uint64_t v[NPT];
#pragma unroll
    for (int j = 0; j < NPT; ++j) v[j] = t + T * j < n ? ll_load(src + t + T * j) : done;
    // While waiting, a thread re-reads only its first entry that is not
    // current; when that one turns current it refreshes all the others.
    // Re-reading every entry each round trip would have all blocks pull
    // tens of MB per microsecond through the fabric while they wait.
    int spin = -1;
    while (true) {
        int first = -1;
#pragma unroll
        for (int j = NPT - 1; j >= 0; --j)
            if (!ll_ready(v[j], epoch)) first = j;
        if (first < 0 || budget == 0) break;
        __builtin_amdgcn_s_sleep(1);
        if (--budget == 0) atomicOr(status, HQ_STEP_SYNC);
        const bool burst = spin >= 0 && spin != first;
#pragma unroll
        for (int j = 0; j < NPT; ++j)
            if (!ll_ready(v[j], epoch) && (burst || j == first)) v[j] = ll_load(src + t + T * j);
        spin = first;
    }
#pragma unroll
    for (int j = 0; j < NPT; ++j) out[j] = (t + T * j < n) ? bits_f32(uint32_t(v[j])) : 0.0f;
    // every load above has been consumed; saying so keeps the compiler from
    // placing a memory wait after the next barrier, where the weight waves'
    // prefetch would then be waited for as well
    wait_all_memory();
}

// ---- block-wide reductions (all 1024 threads call them) ---------------------

// The spec's 256-partial halving tree (partial i + partial i+o, o = 128 ... 1)
// over the partials held by threads 0..255; every thread returns the total.
__device__ __forceinline__ float tree_sum256(float v, float* red)
{
    const int t = opaque_tid();
    if (t < 256) red[t] = v;
    block_sync();
    if (t < 128) red[t] = red[t] + red[t + 128];
    block_sync();
    if (t < 64) {
        const float r = wave_tree_sum64(red[t] + red[t + 64]);
        if (t == 0) red[256] = r;
    }
    block_sync();
    return red[256];
}

__device__ __forceinline__ float block_max16(float v, float* bmax)
{
    const int t = opaque_tid();
    v = wave_max64_all(v);
    if ((t & (kWave - 1)) == 0) bmax[t / kWave] = v;
    block_sync();
    float r = bmax[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) r = fmaxf(r, bmax[w]);
    return r;
}

// Norm weights of this input thread's elements t + 256*j, loaded into
// registers a phase before the RMSNorm that uses them (a load just before
// the poll would delay the poll: a wave's loads complete in order).
template <int NPT>
__device__ __forceinline__ void load_gamma(const float* g, int n, float (&out)[NPT])
{
    const int t = opaque_tid();
#pragma unroll
    for (int j = 0; j < NPT; ++j) out[j] = t + 256 * j < n ? gmem(g)[t + 256 * j] : 0.0f;
}

// Activation prologues.  The phase input is held in registers, element
// t + T*j in out[j] of thread t < T; the int8 result goes to xq in the
// de-interleaved layout, followed by zeros up to npad (the GEMV layouts read
// whole chunk spans: a zero activation makes a padded chunk contribute 0).
// Both end with a barrier; every thread gets the act scale.
// Inputs and norm weights are 0 past n (poll_into, load_gamma), so the
// element loops run unguarded: a zero element adds fmaf(0, 0, ss) = ss to
// the sum of squares, leaves the max unchanged and quantizes to the 0 that
// its xq byte must hold (T*NPT <= kMaxVec keeps those stores inside xq).
// Straight-line code lets the compiler interleave the elements' division
// and rounding chains instead of branching around each one.

// RMSNorm (the spec's 256 strided fmaf partials: T = 256) then quantization.
template <int NPT>
__device__ __forceinline__ float rmsnorm_quant(float (&x)[NPT], int n, const float (&gam)[NPT], float eps,
                                               uint8_t* xq, int npad, float* red, float* bmax,
                                               uint32_t* mk = nullptr)
{
    const int t = opaque_tid();
    const bool mine = t < 256;
    asm volatile("" : "+s"(n));   // keep float(n) from being hoisted out of the layer loop
    static_assert(256 * NPT <= kMaxVec, "xq stores past the buffer");
    float ss = 0.0f;
    if (mine) {
#pragma unroll
        for (int j = 0; j < NPT; ++j) ss = __builtin_fmaf(x[j], x[j], ss);
    }
    SUB_MARK(mk, 0);
    const float total = tree_sum256(ss, red);
    SUB_MARK(mk, 1);
    const float r = __builtin_sqrtf(total / float(n) + eps);
    float amax = 0.0f;
    if (mine) {
#pragma unroll
        for (int j = 0; j < NPT; ++j) x[j] = (x[j] / r) * gam[j];
#pragma unroll
        for (int j = 0; j < NPT; ++j) amax = fmaxf(amax, fabsf(x[j]));
    }
    SUB_MARK(mk, 2);
    amax = fmaxf(block_max16(amax, bmax), 1e-5f);
    SUB_MARK(mk, 3);
    const float inv = 127.0f / amax;
    if (mine) {
#pragma unroll
        for (int j = 0; j < NPT; ++j) xq[xq_offset(t + 256 * j)] = uint8_t(quant_i8(x[j], inv));
    }
    for (int i = n + t; i < npad; i += kThreads) xq[i] = 0;
    SUB_MARK(mk, 4);
    block_sync();
    return amax / 127.0f;
}

// Quantization alone, input held by threads t < T.
template <int T, int NPT>
__device__ __forceinline__ float quantize(const float (&x)[NPT], int n, uint8_t* xq, int npad,
                                          float* bmax)
{
    static_assert(T * NPT <= kMaxVec, "xq stores past the buffer");
    const int t = opaque_tid();
    const bool mine = t < T;
    float amax = 0.0f;
    if (mine) {
#pragma unroll
        for (int j = 0; j < NPT; ++j) amax = fmaxf(amax, fabsf(x[j]));
    }
    amax = fmaxf(block_max16(amax, bmax), 1e-5f);
    const float inv = 127.0f / amax;
    if (mine) {
#pragma unroll
        for (int j = 0; j < NPT; ++j) xq[xq_offset(t + T * j)] = uint8_t(quant_i8(x[j], inv));
    }
    for (int i = n + t; i < npad; i += kThreads) xq[i] = 0;
    block_sync();
    return amax / 127.0f;
}

// ---- weight waves ----------------------------------------------------------
//
// Weights are prefetched two ways.  The o projection (2 chunks per lane) is
// held in registers.  The others are copied straight from HBM into LDS with
// gfx950's 16-byte global->LDS loads, so they take no registers while in
// flight: each weight wave owns a private kWaveStage-byte part of the stage
// buffer, and chunk slot k of the wave sits at sub + k*1024 + lane*16 (the
// load writes its 64 lanes' 16 bytes lane-major).  A wave reuses its part
// phase after phase (qkv slots 0-2, gate_up 0-9, down 0-4) only after its own
// dot has read the previous contents; the attention work area aliases the
// stage buffer and is bracketed by block barriers.

// Rows [r0, r1) of W (K columns), RPW = 64/LPR rows per weight wave; wave
// ww owns rows r0 + ww*RPW .. + RPW-1, lane li of a row reads chunks
// li + (J0 + j)*LPR (clamped into the row; a clamped chunk meets zero
// activations).  Returns the epilogue row scale (lane r < RPW: row r).
__device__ __forceinline__ int wave_row(int r0, int r1, int ww, int lane, int lpr)
{
    return min(r0 + ww * (kWave / lpr) + lane / lpr, r1 - 1);
}

// One 16-byte global->LDS load per lane from W + off (W uniform, off a
// 32-bit byte offset) into lds + 16*lane.  Written as asm: the compiler's
// own tracking of this instruction made later, unrelated instructions wait
// for it (they reuse its offset register).  Loads the compiler does not see
// can only make its other waits longer, never too short; the staged data is
// read only after an explicit wait for all of the wave's memory operations.
__device__ __forceinline__ void dma16(const uint8_t* W, uint32_t off, uint8_t* lds)
{
    const uint32_t m = __builtin_amdgcn_readfirstlane(
        uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t*)lds)));
    uint32_t saved;   // m0 is reserved to the compiler: restore it
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
                 "global_load_lds_dwordx4 %2, %3\n\ts_nop 0\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(m), "v"(off), "s"(uniform_ptr(W))
                 : "memory");
}

// LDS prefetch of plain rows (chunks li + j*LPR) into chunk slots SLOT0..
// of the wave's stage part (row scales are read at the dot, see row_scale).
template <int LPR, int MAXC, int SLOT0 = 0>
__device__ __forceinline__ void stage_rows(uint8_t* stage, bool active, const uint8_t* W, int r0, int r1,
                                           int K, int ww)
{
    constexpr int RPW = kWave / LPR;
    if (!active || r0 + ww * RPW >= r1) return;
    const int lane = lane_id();
    const int nch = K >> 5;
    const int li = lane % LPR;
    const uint32_t rowoff = uint32_t(wave_row(r0, r1, ww, lane, LPR)) * uint32_t(K >> 1);
    uint8_t* sub = stage + __builtin_amdgcn_readfirstlane(ww) * kWaveStage;
#pragma unroll
    for (int j = 0; j < MAXC; ++j)
        dma16(W, rowoff + uint32_t(min(li + j * LPR, nch - 1)) * 16, sub + (SLOT0 + j) * 1024);
}

// Waits until at most N of the wave's memory operations are outstanding
// (they complete in issue order): a dot waits for its own weights but not
// for the prefetch issued after them.  Only weight waves use it, and they
// issue no other memory operations after the prefetch they skip.
template <int N>
__device__ __forceinline__ void wait_memory_but()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One 4-byte global->LDS load per lane from S + off into lds + 4*lane.
__device__ __forceinline__ void dma4(const float* S, uint32_t off, float* lds)
{
    const uint32_t m = __builtin_amdgcn_readfirstlane(
        uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) float*)lds)));
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
                 "global_load_lds_dword %2, %3\n\ts_nop 0\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(m), "v"(off), "s"(uniform_ptr(S))
                 : "memory");
}

// Row scales travel with their weights: lane i of weight wave ww copies the
// scale of the wave's row min(i, RPW-1) into scl[ww][i] (read after the
// dot's wait for the wave's global->LDS loads).
template <int LPR>
__device__ __forceinline__ void stage_scales(float (*scl)[kWave], bool active, const float* S, int r0, int r1,
                                             int ww)
{
    constexpr int RPW = kWave / LPR;
    if (!active || r0 + ww * RPW >= r1) return;
    const int row = min(r0 + ww * RPW + min(lane_id(), RPW - 1), r1 - 1);
    dma4(S, uint32_t(row) * 4u, scl[__builtin_amdgcn_readfirstlane(ww)]);
}

// SwiGLU scales: lanes 0-3 the gate rows of the wave's four pairs, lanes 4-7
// the matching up rows (I + pair); the others repeat them.
__device__ __forceinline__ void stage_pair_scales(float (*scl)[kWave], bool active, const float* S, int p0,
                                                  int p1, int I, int ww)
{
    if (!active || p0 + ww * 4 >= p1) return;
    const int lane = lane_id();
    const int pair = min(p0 + ww * 4 + (lane & 3), p1 - 1);
    const int row = (lane & 4) ? I + pair : pair;
    dma4(S, uint32_t(row) * 4u, scl[__builtin_amdgcn_readfirstlane(ww)]);
}

// LDS prefetch of SwiGLU rows: pairs [p0, p1) of the I gate rows; weight
// wave ww owns pairs p0 + 4*ww .. +3, its lane groups 0-3 read the gate rows
// and 4-7 the matching up rows (row I + pair); chunks li + (J0 + j)*8.
template <int MAXC, int J0>
__device__ __forceinline__ void stage_pairs(uint8_t* stage, bool active, const uint8_t* W, int p0, int p1,
                                            int I, int K, int ww)
{
    if (!active || p0 + ww * 4 >= p1) return;
    const int lane = lane_id();
    const int nch = K >> 5;
    const int rsel = lane >> 3;
    const int pair = min(p0 + ww * 4 + (rsel & 3), p1 - 1);
    const int row = rsel < 4 ? pair : I + pair;
    const int li = lane & 7;
    const uint32_t rowoff = uint32_t(row) * uint32_t(K >> 1);
    uint8_t* sub = stage + __builtin_amdgcn_readfirstlane(ww) * kWaveStage;
#pragma unroll
    for (int j = 0; j < MAXC; ++j)
        dma16(W, rowoff + uint32_t(min(li + (J0 + j) * 8, nch - 1)) * 16, sub + (J0 + j) * 1024);
}

// 16 * partial dot product of this lane's NC staged chunks (slots SLOT0..,
// chunks li + j*LPR) with the LDS activations, two chunks at
// a time: loading all slots and activations up front would need ~30 LDS
// reads' worth of registers.  The caller has waited for the wave's
// global->LDS loads.
template <int LPR, int NC, int SLOT0 = 0>
__device__ __forceinline__ int staged_dot(const uint8_t* stage, const uint8_t* xq, int ww)
{
    const int lane = lane_id();
    const int li = lane % LPR;
    const uint8_t* sub = stage + ww * kWaveStage + SLOT0 * 1024 + lane * 16;
    int a0 = 0, a1 = 0, a2 = 0, a3 = 0;
#pragma unroll
    for (int j = 0; j < NC; j += 2) {
        const uint4 w0 = *reinterpret_cast<const uint4*>(sub + j * 1024);
        dot_chunk(w0, xq + (li + j * LPR) * 32, a0, a1);
        if (j + 1 < NC) {
            const uint4 w1 = *reinterpret_cast<const uint4*>(sub + (j + 1) * 1024);
            dot_chunk(w1, xq + (li + (j + 1) * LPR) * 32, a2, a3);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    return (a0 + a1) + (a2 + a3);
}

// Register prefetch of SwiGLU chunks J0 .. J0+NR-1 (same lane mapping as
// stage_pairs).  Ordinary loads: the compiler waits for them at their use.
template <int NR, int J0>
__device__ __forceinline__ void load_pairs(uint4 (&w)[NR], bool active, const uint8_t* W, int p0, int p1, int I,
                                           int K, int ww)
{
    if (!active || p0 + ww * 4 >= p1) return;
    const int lane = lane_id();
    const int nch = K >> 5;
    const int rsel = lane >> 3;
    const int pair = min(p0 + ww * 4 + (rsel & 3), p1 - 1);
    const int row = rsel < 4 ? pair : I + pair;
    const int li = lane & 7;
    const uint8_t* base = W + size_t(row) * size_t(K >> 1);
#pragma unroll
    for (int j = 0; j < NR; ++j) w[j] = load_w16(base + size_t(min(li + (J0 + j) * 8, nch - 1)) * 16);
}

// staged_dot over NS staged chunks (slots 0..NS-1) followed by NR chunks
// held in registers (chunk indices NS..NS+NR-1).
template <int LPR, int NS, int NR>
__device__ __forceinline__ int staged_reg_dot(const uint8_t* stage, const uint4 (&w)[NR], const uint8_t* xq,
                                              int ww)
{
    const int lane = lane_id();
    const int li = lane % LPR;
    int a0 = 0, a1 = 0, a2 = 0, a3 = 0;
#pragma unroll
    for (int j = 0; j < NR; j += 2) {
        dot_chunk(w[j], xq + (li + (NS + j) * LPR) * 32, a2, a3);
        if (j + 1 < NR) dot_chunk(w[j + 1], xq + (li + (NS + j + 1) * LPR) * 32, a0, a1);
        __builtin_amdgcn_sched_barrier(0);
    }
    return staged_dot<LPR, NS>(stage, xq, ww) + ((a0 + a1) + (a2 + a3));
}

// Lane r < COUNT receives the accumulator of the wave's row FIRST + r
// (FIRST + COUNT <= 64 / LPR).
template <int LPR, int FIRST, int COUNT>
__device__ __forceinline__ int rows_acc(int part, int lane)
{
    static_assert(FIRST + COUNT <= kWave / LPR, "row outside the wave");
    int acc = 0;
#pragma unroll
    for (int r = 0; r < COUNT; ++r) {
        const int t = row_isum<LPR>(part, FIRST + r) >> 4;
        if (lane == r) acc = t;
    }
    return acc;
}

// ---- attention (P2) ----------------------------------------------------------

struct AttnLds {
    float raw[(kG + 2) * kD];      // polled q heads, k, v of this kv head
    float qn[kD], kn[kD], cs[kD / 2], sn[kD / 2];
    alignas(16) float q[kG][kD];
    uint16_t k[kAttnChunk * kRow];
    uint16_t v[kAttnChunk * kRow];
    uint16_t kc[kD], vc[kD];
    alignas(16) float e[kG][kAttnChunk];
    float m[kG][kCPB], l[kG][kCPB];
    float alpha[kG][kCPB], inv_l[kG];
    alignas(16) float o[kCPB][kG][kD];
};

// K/V of chunk rows [t0, t0 + tn) into registers: 64 rows x 16 groups of
// 8 halves, one 16-byte K and V group per thread of the block.  The current
// position's row is skipped (it comes from kc/vc).
__device__ __forceinline__ void load_kv_chunk(const uint16_t* keys, const uint16_t* vals, int stride,
                                              size_t kv_off, int t0, int tn, int skip_t,
                                              uint4& kreg, uint4& vreg)
{
    const int id = opaque_tid();
    const int t = id >> 4;
    const int d8 = id & 15;
    const bool ok = t < tn && t != skip_t;
    const size_t off = size_t(t0 + t) * size_t(stride) + kv_off + size_t(d8) * 8;
    kreg = ok ? *reinterpret_cast<const uint4*>(keys + off) : make_uint4(0, 0, 0, 0);
    vreg = ok ? *reinterpret_cast<const uint4*>(vals + off) : make_uint4(0, 0, 0, 0);
}

// One attention work item (kv head, split) of layer l, run by the whole
// block with uniform control flow.  Same arithmetic as attention_kernel's
// STEP mode (hq_attention.hip).
__device__ void attention_item(const EngineParams& p, const float* q_norm, const float* k_norm, int l, int item, int nsplit,
                               int n, int nc, int pos, uint32_t epoch_qkv, uint32_t epoch_att,
                               AttnLds& A, int& last, unsigned& budget, uint32_t* atr)
{
#ifdef HQ_ENGINE_TRACE
#define ATT_MARK(k)                                                                                 \
    do {                                                                                            \
        const int t_ = opaque_tid();                                                                \
        if ((t_ & (kWave - 1)) == 0 && l >= kTraceL0 && l < kTraceL0 + 4)                           \
            atr[((l - kTraceL0) * 16 + (k)) * 16 + t_ / kWave] = uint32_t(wall_clock64());          \
    } while (0)
#else
#define ATT_MARK(k) do { (void)atr; } while (0)
#endif
    // A aliases the weight waves' stage buffer: wait until every wave is
    // done with its staged qkv weights
    block_sync();
    ATT_MARK(0);
    const int tid = opaque_tid();
    const int wave = tid / kWave;
    const int lane = tid & (kWave - 1);
    const int G = p.G;
    const int kvh = item / nsplit;
    const int split = item % nsplit;
    const int c_begin = split * kCPB;
    const int c_end = min(nc, c_begin + kCPB);
    const bool last_split = split == nsplit - 1;
    const int cur_chunk = nc - 1;
    const size_t kv_off = size_t(kvh) * kD;
    uint16_t* keys = p.keys + size_t(l) * size_t(p.kv_layer);
    uint16_t* vals = p.values + size_t(l) * size_t(p.kv_layer);
    constexpr int C = kAttnChunk;

    // the first chunk's K/V are loaded by every thread before the q/k/v poll
    // (the weight waves have only the o-projection prefetch in flight here)
    uint4 kreg, vreg;
    {
        const int t0 = c_begin * C;
        load_kv_chunk(keys, vals, p.kv_stride, kv_off, t0, min(C, n - t0),
                      c_begin == cur_chunk ? pos - t0 : -1, kreg, vreg);
    }
    if (tid < kIThreads) {
        if (tid < kD) {
            A.qn[tid] = gmem(q_norm)[tid];
            A.kn[tid] = gmem(k_norm)[tid];
        } else {
            const int i = tid - kD;
            if (i < kD / 2) A.cs[i] = p.rope_cos[size_t(pos) * (kD / 2) + i];
            else A.sn[i - kD / 2] = p.rope_sin[size_t(pos) * (kD / 2) + (i - kD / 2)];
        }
    }
    // q rows of the G heads, then k and v of this kv head: entry e of the
    // item's ne inputs sits at ll_qkv[qkv_src(e)]
    const int nq = G * kD;
    const int ne = nq + 2 * kD;
    const int qd = p.heads * kD;
    auto qkv_src = [&](int e) {
        return e < nq ? kvh * nq + e
                      : (e < nq + kD ? qd + kvh * kD + (e - nq) : qd + p.kv_heads * kD + kvh * kD + (e - nq - kD));
    };
    if (tid < kWave) {   // wave 0 watches 64 spread entries (see watch_spread)
        const int src = qkv_src(((tid + 1) * ne) / kWave - 1);
        uint64_t w = ll_load(p.ll_qkv + src);
        while (!ll_ready(w, epoch_qkv) && budget != 0) {
            __builtin_amdgcn_s_sleep(1);
            if (--budget == 0) atomicOr(p.status, HQ_STEP_SYNC);
            w = ll_load(p.ll_qkv + src);
        }
    }
    block_sync();
    if (tid < kIThreads) {
        uint64_t v[3];
        int src[3];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            src[j] = qkv_src(min(tid + kIThreads * j, ne - 1));
            v[j] = ll_load(p.ll_qkv + src[j]);
        }
        int spin = -1;   // as in poll_into: spin on one entry, then refresh the rest
        while (true) {
            int first = -1;
#pragma unroll
            for (int j = 2; j >= 0; --j)
                if (tid + kIThreads * j < ne && !ll_ready(v[j], epoch_qkv)) first = j;
            if (first < 0 || budget == 0) break;
            __builtin_amdgcn_s_sleep(1);
            if (--budget == 0) atomicOr(p.status, HQ_STEP_SYNC);
            const bool burst = spin >= 0 && spin != first;
#pragma unroll
            for (int j = 0; j < 3; ++j)
                if (tid + kIThreads * j < ne && !ll_ready(v[j], epoch_qkv) && (burst || j == first))
                    v[j] = ll_load(p.ll_qkv + src[j]);
            spin = first;
        }
#pragma unroll
        for (int j = 0; j < 3; ++j)
            if (tid + kIThreads * j < ne) A.raw[tid + kIThreads * j] = bits_f32(uint32_t(v[j]));
    }
    block_sync();

    ATT_MARK(2);
    // per-head RMSNorm + RoPE of q; k (norm + RoPE) and v appended as fp16
    if (wave < G) {
        const float x0 = A.raw[wave * kD + lane], x1 = A.raw[wave * kD + lane + 64];
        float s = __builtin_fmaf(x0, x0, 0.0f);
        s = __builtin_fmaf(x1, x1, s);
        const float ss = wave_tree_sum64_all(s);
        const float r = __builtin_sqrtf(ss / float(kD) + p.eps);
        const float y0 = (x0 / r) * A.qn[lane];
        const float y1 = (x1 / r) * A.qn[lane + 64];
        const float c0 = A.cs[lane], s0 = A.sn[lane];
        A.q[wave][lane] = y0 * c0 - y1 * s0;
        A.q[wave][lane + 64] = y1 * c0 + y0 * s0;
    } else if (last_split && wave == G) {
        const float x0 = A.raw[G * kD + lane], x1 = A.raw[G * kD + lane + 64];
        float s = __builtin_fmaf(x0, x0, 0.0f);
        s = __builtin_fmaf(x1, x1, s);
        const float ss = wave_tree_sum64_all(s);
        const float r = __builtin_sqrtf(ss / float(kD) + p.eps);
        const float y0 = (x0 / r) * A.kn[lane];
        const float y1 = (x1 / r) * A.kn[lane + 64];
        const float c0 = A.cs[lane], s0 = A.sn[lane];
        A.kc[lane] = f32_to_f16(y0 * c0 - y1 * s0);
        A.kc[lane + 64] = f32_to_f16(y1 * c0 + y0 * s0);
    } else if (last_split && wave == G + 1) {
        A.vc[lane] = f32_to_f16(A.raw[(G + 1) * kD + lane]);
        A.vc[lane + 64] = f32_to_f16(A.raw[(G + 1) * kD + lane + 64]);
    }
    block_sync();
    // the fp16 k/v of this position go to the cache from the input waves
    // (weight waves issue no global stores: see block_sync and dma16)
    if (last_split && tid < 2 * kD) {
        if (tid < kD) keys[size_t(pos) * size_t(p.kv_stride) + kv_off + tid] = A.kc[tid];
        else vals[size_t(pos) * size_t(p.kv_stride) + kv_off + (tid - kD)] = A.vc[tid - kD];
    }

    ATT_MARK(3);
    const int grp = tid >> 4;        // position of the chunk this lane group scores
    const int l16 = tid & 15;
    const float scale = 1.0f / __builtin_sqrtf(float(kD));
    const int vh = tid >> 7;         // V accumulation: (head, dim) per thread
    const int vd = tid & (kD - 1);

#pragma unroll 1
    for (int ci = 0; ci < kCPB; ++ci) {
        const int c = c_begin + ci;
        if (c >= c_end) break;
        const int t0 = c * C;
        const int tn = min(C, n - t0);
        {
            const int t = tid >> 4;
            const int d8 = tid & 15;
            if (t < tn) {
                uint4 kv = kreg, vv = vreg;
                if (c == cur_chunk && t0 + t == pos) {
                    kv = *reinterpret_cast<const uint4*>(A.kc + d8 * 8);
                    vv = *reinterpret_cast<const uint4*>(A.vc + d8 * 8);
                }
                *reinterpret_cast<uint4*>(A.k + t * kRow + d8 * 8) = kv;
                *reinterpret_cast<uint4*>(A.v + t * kRow + d8 * 8) = vv;
            }
        }
        block_sync();
        if (ci == 0) ATT_MARK(4);
        if (c + 1 < c_end) {
            const int t1 = t0 + C;
            load_kv_chunk(keys, vals, p.kv_stride, kv_off, t1, min(C, n - t1),
                          c + 1 == cur_chunk ? pos - t1 : -1, kreg, vreg);
        }
        __builtin_amdgcn_sched_barrier(0);

        // scores: 16 lanes per position, 8 dims per lane
        if (grp < tn) {
            float k[8];
            const uint16_t* kr = A.k + grp * kRow + l16 * 8;
#pragma unroll
            for (int j = 0; j < 8; ++j) k[j] = f16_to_f32(kr[j]);
#pragma unroll
            for (int h = 0; h < kG; ++h) {
                if (h < G) {
                    // q from LDS: with one position per lane group the
                    // query is used once per chunk
                    const float4 qa = *reinterpret_cast<const float4*>(&A.q[h][l16 * 8]);
                    const float4 qb = *reinterpret_cast<const float4*>(&A.q[h][l16 * 8 + 4]);
                    const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
                    float pp = 0.0f;
#pragma unroll
                    for (int j = 0; j < 8; ++j) pp = __builtin_fmaf(qv[j], k[j], pp);
                    const float dot = row_tree_sum16(pp);
                    if (l16 == 0) A.e[h][grp] = dot * scale;
                }
            }
        } else if (l16 == 0) {
#pragma unroll
            for (int h = 0; h < kG; ++h)
                if (h < G) A.e[h][grp] = -__builtin_inff();
        }
        block_sync();
        if (ci == 0) ATT_MARK(5);

        if (wave < G) {
            const float sc = A.e[wave][lane];
            const float m = wave_max64_all(sc);
            const float e = (lane < tn) ? spec_expf(sc - m) : 0.0f;
            const float ls = wave_tree_sum64(e);
            A.e[wave][lane] = e;
            if (lane == 0) { A.m[wave][ci] = m; A.l[wave][ci] = ls; }
        }
        block_sync();
        if (ci == 0) ATT_MARK(6);

        if (vh < G) {
            // o = fmaf chain over ascending positions; a full chunk reads 16
            // positions ahead of their fmas, so the chain waits on LDS once
            // per 16 positions instead of once per 8
            float o = 0.0f;
            if (tn == C) {
#pragma unroll
                for (int i0 = 0; i0 < C; i0 += 16) {
                    float vv[16], ee[16];
#pragma unroll
                    for (int j = 0; j < 16; j += 4) {
                        const float4 e4 = *reinterpret_cast<const float4*>(&A.e[vh][i0 + j]);
                        ee[j] = e4.x; ee[j + 1] = e4.y; ee[j + 2] = e4.z; ee[j + 3] = e4.w;
                    }
#pragma unroll
                    for (int j = 0; j < 16; ++j) vv[j] = f16_to_f32(A.v[(i0 + j) * kRow + vd]);
#pragma unroll
                    for (int j = 0; j < 16; ++j) o = __builtin_fmaf(ee[j], vv[j], o);
                }
            } else {
                int i = 0;
#pragma unroll 1
                for (; i + 8 <= tn; i += 8) {
                    float vv[8], ee[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        vv[j] = f16_to_f32(A.v[(i + j) * kRow + vd]);
                        ee[j] = A.e[vh][i + j];
                    }
#pragma unroll
                    for (int j = 0; j < 8; ++j) o = __builtin_fmaf(ee[j], vv[j], o);
                }
#pragma unroll 1
                for (; i < tn; ++i) o = __builtin_fmaf(A.e[vh][i], f16_to_f32(A.v[i * kRow + vd]), o);
            }
            A.o[ci][vh][vd] = o;
        }
        block_sync();
        if (ci == 0) ATT_MARK(7);
    }
    ATT_MARK(8);

    const int nmine = c_end - c_begin;
    if (nsplit == 1) {
        // the combine weights a_c = exp(m_c - M) and 1/L depend on the head
        // only: one lane per head computes them (same operations, same bits)
        if (tid < G) {
            float M = -__builtin_inff();
            for (int ci = 0; ci < nmine; ++ci) M = fmaxf(M, A.m[tid][ci]);
            float L = 0.0f;
            for (int ci = 0; ci < nmine; ++ci) {
                const float al = spec_expf(A.m[tid][ci] - M);
                A.alpha[tid][ci] = al;
                L = __builtin_fmaf(al, A.l[tid][ci], L);
            }
            A.inv_l[tid] = 1.0f / L;
        }
        block_sync();
        ATT_MARK(9);
        if (tid < kIThreads) {
            for (int pr = tid; pr < G * kD; pr += kIThreads) {
                const int h = pr >> 7, d = pr & (kD - 1);
                float O = 0.0f;
                for (int ci = 0; ci < nmine; ++ci) O = __builtin_fmaf(A.alpha[h][ci], A.o[ci][h][d], O);
                ll_store(p.ll_att + size_t(kvh * G + h) * kD + d, O * A.inv_l[h], epoch_att);
            }
        }
        block_sync();
        ATT_MARK(10);
        return;
    }

    // several splits: the input waves publish this item's chunk partials,
    // and the last split of the kv head to arrive combines all of them
    const int pstride = kD + 2;
    if (tid < kIThreads) {
        for (int pr = tid; pr < G * kD; pr += kIThreads) {
            const int h = pr >> 7, d = pr & (kD - 1);
            for (int ci = 0; ci < nmine; ++ci) {
                float* pp = p.part + (size_t(kvh * G + h) * p.max_chunks + (c_begin + ci)) * pstride;
                publish_f(pp + 2 + d, A.o[ci][h][d]);
                if (d == 0) { publish_f(pp, A.m[h][ci]); publish_f(pp + 1, A.l[h][ci]); }
            }
        }
        wait_all_memory();
    }
    block_sync();
    if (tid == 0) last = atomicAdd(p.counters + kvh, 1) == nsplit - 1;
    block_sync();
    if (!last) return;     // block-uniform; `last` lies outside the stage buffer
    // the ticket is reset (and the reset completed) before any output is
    // published: the next layer's arrivals depend on those outputs
    if (tid == 0) {
        publish_i(p.counters + kvh, 0);
        wait_all_memory();
    }
    block_sync();
    if (tid < kIThreads) {
        for (int pr = tid; pr < G * kD; pr += kIThreads) {
            const int h = pr >> 7, d = pr & (kD - 1);
            const float* base = p.part + size_t(kvh * G + h) * p.max_chunks * pstride;
            float M = -__builtin_inff();
            for (int cc = 0; cc < nc; ++cc) M = fmaxf(M, read_f(base + size_t(cc) * pstride));
            float L = 0.0f, O = 0.0f;
            for (int cc = 0; cc < nc; ++cc) {
                const float* pc = base + size_t(cc) * pstride;
                const float al = spec_expf(read_f(pc) - M);
                L = __builtin_fmaf(al, read_f(pc + 1), L);
                O = __builtin_fmaf(al, read_f(pc + 2 + d), O);
            }
            ll_store(p.ll_att + size_t(kvh * G + h) * kD + d, O * (1.0f / L), epoch_att);
        }
    }
    block_sync();
}

}  // namespace

__global__ __launch_bounds__(eng::kThreads) void engine_kernel(EngineParams p)
{
    __shared__ __align__(16) uint8_t xq_s[kMaxVec];
    __shared__ float red[260];
    __shared__ float bmax[kWaves];
    __shared__ float xown_s[kMaxOwn];
    __shared__ float res_s[kMaxRes];   // a GEMV phase's outputs, published by the input waves
    __shared__ int last_s;
    // weight stage (kWaveStage bytes per weight wave); the attention work
    // area of P2 aliases it
    __shared__ __align__(16) uint8_t stage_s[kWWaves * kWaveStage];
    // row scales staged with the weights: [0] qkv then o, [1] gate_up then down
    __shared__ float scl_s[3][kWWaves][kWave];   // qkv then o | gate_up | down
    static_assert(sizeof(AttnLds) <= sizeof(stage_s), "attention area larger than the stage");
    AttnLds& A = *reinterpret_cast<AttnLds*>(stage_s);
    // The layer table, copied once.  Read from global memory inside the
    // loop, its pointers would be vector loads (the kernel writes global
    // memory, so they cannot be scalar loads), and a weight wave's wait for
    // one would also wait for every weight load it has in flight.
    __shared__ hq_layer lay_s[kMaxLayers];
#ifdef HQ_ENGINE_TRACE
    __shared__ uint32_t trace_s[4 * 16 * 16];
    __shared__ uint32_t atr_s[4 * 16 * 16];
    __shared__ uint32_t sub_s[4 * 16 * 16];
    for (int i = threadIdx.x; i < 4 * 16 * 16; i += kThreads) atr_s[i] = sub_s[i] = 0;
#else
    uint32_t* const atr_s = nullptr;
#endif

    const int tid = threadIdx.x;
    const bool iw = tid < kIThreads;
    const int ww = tid / kWave - kIThreads / kWave;
    const int b = blockIdx.x;
    const int NB = gridDim.x;

    const int pos = *p.position;
    if (pos < 0 || pos >= p.capacity) {
        if (b == 0 && tid == 0) atomicOr(p.status, HQ_STEP_FULL);
        return;
    }
    const uint32_t base = *p.epoch;
    const int H = p.H, I = p.I;
    const int qd = p.heads * kD;
    const int h0 = split_begin(H, b, NB), h1 = split_begin(H, b + 1, NB);
    const int q0 = split_begin(p.qkv_rows, b, NB), q1 = split_begin(p.qkv_rows, b + 1, NB);
    const int g0 = split_begin(I, b, NB), g1 = split_begin(I, b + 1, NB);
    if (tid < h1 - h0) xown_s[tid] = p.x[h0 + tid];
    {
        constexpr int kWords = sizeof(hq_layer) / sizeof(uint64_t);
        const uint64_t* src = reinterpret_cast<const uint64_t*>(p.layers);
        uint64_t* dst = reinterpret_cast<uint64_t*>(lay_s);
        for (int i = tid; i < p.L * kWords; i += kThreads) dst[i] = src[i];
    }
    block_sync();
    unsigned budget = kPollBudget;

    const int n = pos + 1;
    const int nc = (n + kAttnChunk - 1) / kAttnChunk;
    const int nsplit = (nc + kCPB - 1) / kCPB;
    const int items = p.kv_heads * nsplit;

    // Weight prefetch schedule (the phases in between are its lead time);
    // a wave overwrites stage slots only after its own dot has read them.
    // Loads issued just before a hand-off would sit in the CU's memory queue
    // ahead of the poll, so the gate_up and down halves wait until their
    // phase's input has been read:
    //   qkv      slots 0-2   after the P5 input read of the previous layer
    //   o        slots 5-6   end of P2
    //   gate_up  slots 0-4   end of P2, its second half in registers (also
    //            loaded at the end of P2, used at P4)
    //   down     slots 5-9   after the P4 input read
    stage_rows<kQkvLPR, kQkvMAXC>(stage_s, !iw, lay_s[0].qkv, q0, q1, H, ww);
    stage_scales<kQkvLPR>(scl_s[0], !iw, lay_s[0].qkv_scales, q0, q1, ww);
    float gin[kHidNPT] = {};   // input_norm of the coming P1 (input waves)
    if (iw) load_gamma(lay_s[0].input_norm, H, gin);

#pragma unroll 1
    for (int l = 0; l < p.L; ++l) {
        // thread-derived values re-derived per layer (see opaque_tid)
        const int tid = opaque_tid();
        const bool iw = tid < kIThreads;
        const int ww = tid / kWave - kIThreads / kWave;
        const hq_layer& Ly = lay_s[l];
        const uint32_t E = base + 5u * uint32_t(l);
        const bool final_layer = l + 1 == p.L;

        ENG_MARK(0);
        // ---- P1: RMSNorm(input) -> quant -> qkv -------------------------------
        // each phase input is a fresh, fully initialised array: nothing of it
        // stays live into the next phase on any path
        float xin[kHidNPT] = {};
        if (l > 0) watch_spread(p.ll_x5, H, E, budget, p.status);
        block_sync();
        if (iw) {
            if (l == 0) {
#pragma unroll
                for (int j = 0; j < kHidNPT; ++j)
                    xin[j] = tid + kIThreads * j < H ? p.x[tid + kIThreads * j] : 0.0f;
            } else {
                poll_into<kIThreads, kHidNPT>(p.ll_x5, H, E, xin, budget, p.status);
            }
        }
        ENG_MARK(1);
        block_sync();
        ENG_MARK(2);
#ifdef HQ_ENGINE_TRACE
        uint32_t* const mk = l >= kTraceL0 && l < kTraceL0 + 4 ? sub_s + (l - kTraceL0) * 256 : nullptr;
#else
        uint32_t* const mk = nullptr;
#endif
        float act = rmsnorm_quant(xin, H, gin, p.eps, xq_s, kQkvLPR * kQkvMAXC * 32, red, bmax);
        ENG_MARK(3);
        if (!iw && q0 + ww * 2 < q1) {
            wait_all_memory();   // the staged qkv weights and scales
            const int part = staged_dot<kQkvLPR, kQkvMAXC>(stage_s, xq_s, ww);
            const int acc = rows_acc<kQkvLPR, 0, 2>(part, lane_id());
            const int row = q0 + ww * 2 + lane_id();
            if (lane_id() < 2 && row < q1) res_s[row - q0] = (float(acc) * act) * scl_s[0][ww][lane_id()];
        }
        block_sync();
        publish_rows(res_s, p.ll_qkv + q0, q1 - q0, E + 1);
        ENG_MARK(4);

        // ---- P2: attention --------------------------------------------------
        for (int it = b; it < items; it += NB)
            attention_item(p, uniform_ptr(Ly.q_norm), uniform_ptr(Ly.k_norm), l, it, nsplit, n, nc, pos,
                           E + 1, E + 2, A, last_s, budget, atr_s);
        // everything the attention loaded has been consumed; saying so keeps
        // the compiler's waits for those loads from landing after the weight
        // prefetch below, where they would wait for it too
        wait_all_memory();
        ENG_MARK(5);
        stage_rows<kOLPR, kOMAXC, 5>(stage_s, !iw, Ly.o, h0, h1, qd, ww);
        stage_scales<kOLPR>(scl_s[0], !iw, Ly.o_scales, h0, h1, ww);
        stage_pairs<kGuHalf, 0>(stage_s, !iw, Ly.gate_up, g0, g1, I, H, ww);
        stage_pair_scales(scl_s[1], !iw, Ly.gate_up_scales, g0, g1, I, ww);
        uint4 gub[kGuHalf];   // second gate_up half (weight waves), used at P4
#pragma unroll
        for (int j = 0; j < kGuHalf; ++j) gub[j] = make_uint4(0, 0, 0, 0);
        load_pairs<kGuHalf, kGuHalf>(gub, !iw, Ly.gate_up, g0, g1, I, H, ww);

        // ---- P3: quant -> o -> residual ----------------------------------------
        float att[kAttNPT] = {};
        float gpost[kHidNPT] = {};   // post_norm for P4, loaded once the poll is done
        watch_spread(p.ll_att, qd, E + 2, budget, p.status);
        SUB_MARK(mk, 9);
        block_sync();
        SUB_MARK(mk, 10);
        if (iw) {
            poll_into<kIThreads, kAttNPT>(p.ll_att, qd, E + 2, att, budget, p.status);
            load_gamma(Ly.post_norm, H, gpost);
        }
        ENG_MARK(6);
        block_sync();
        ENG_MARK(7);
        act = quantize<kIThreads, kAttNPT>(att, qd, xq_s, kOLPR * kOMAXC * 32, bmax);
        if (!iw && h0 + ww < h1) {
            // the staged o weights and scale, not the gate_up loads behind
            // them (kGuHalf staged + 1 scale + kGuHalf register loads when the
            // wave has pairs)
            if (g0 + ww * 4 < g1) wait_memory_but<2 * kGuHalf + 1>();
            else wait_all_memory();
            const int part = staged_dot<kOLPR, kOMAXC, 5>(stage_s, xq_s, ww);
            const int acc = rows_acc<kOLPR, 0, 1>(part, lane_id());
            if (lane_id() == 0) {
                const float xn = xown_s[ww] + (float(acc) * act) * scl_s[0][ww][0];
                xown_s[ww] = xn;
                res_s[ww] = xn;
            }
        }
        block_sync();
        publish_rows(res_s, p.ll_x3 + h0, h1 - h0, E + 3);
        ENG_MARK(8);

        // ---- P4: RMSNorm(post) -> quant -> gate_up -> SwiGLU -----------------------
        float xpost[kHidNPT] = {};
        watch_spread(p.ll_x3, H, E + 3, budget, p.status);
        SUB_MARK(mk, 11);
        block_sync();
        SUB_MARK(mk, 12);
        if (iw) poll_into<kIThreads, kHidNPT>(p.ll_x3, H, E + 3, xpost, budget, p.status);
        ENG_MARK(9);
        block_sync();
        ENG_MARK(10);
        // The register half of gate_up landed during P3; waiting for it here,
        // before the down prefetch is issued, settles the compiler's own wait
        // for those registers (otherwise placed at their use, where it would
        // also wait for the down prefetch, which the compiler cannot see).
        if (!iw) wait_all_memory();
        stage_rows<kDownLPR, kDownMAXC, 5>(stage_s, !iw, Ly.down, h0, h1, I, ww);
        stage_scales<kDownLPR>(scl_s[2], !iw, Ly.down_scales, h0, h1, ww);
        act = rmsnorm_quant(xpost, H, gpost, p.eps, xq_s, kGuLPR * 2 * kGuHalf * 32, red, bmax, mk);
        if (!iw && g0 + ww * 4 < g1) {
            // the staged gate_up half, its scales and the register half, not
            // the down prefetch behind them (kDownMAXC + 1 loads)
            SUB_MARK(mk, 5);
            if (h0 + ww < h1) wait_memory_but<kDownMAXC + 1>();
            else wait_all_memory();
            SUB_MARK(mk, 6);
            const float sg = scl_s[1][ww][lane_id() & 3];
            const float su = scl_s[1][ww][4 + (lane_id() & 3)];
            const int part = staged_reg_dot<kGuLPR, kGuHalf, kGuHalf>(stage_s, gub, xq_s, ww);
            const int acc = rows_acc<kGuLPR, 0, 4>(part, lane_id());
            const int acc_up = rows_acc<kGuLPR, 4, 4>(part, lane_id());
            const int pair = g0 + ww * 4 + lane_id();
            if (lane_id() < 4 && pair < g1) {
                const float g = (float(acc) * act) * sg;
                const float u = (float(acc_up) * act) * su;
                const float t = 1.0f + spec_expf(-g);
                res_s[pair - g0] = (g / t) * u;
            }
            SUB_MARK(mk, 7);
        }
        block_sync();
        SUB_MARK(mk, 8);
        publish_rows(res_s, p.ll_act + g0, g1 - g0, E + 4);
        ENG_MARK(11);

        // ---- P5: quant -> down -> residual -------------------------------------
        // all waves poll: the weight waves' down prefetch (issued just now)
        // lands well within the hand-off time
        float av[kActNPT] = {};
        watch_spread(p.ll_act, I, E + 4, budget, p.status);
        SUB_MARK(mk, 13);
        block_sync();
        SUB_MARK(mk, 14);
        poll_into<kThreads, kActNPT>(p.ll_act, I, E + 4, av, budget, p.status);
        if (iw && !final_layer) load_gamma(lay_s[l + 1].input_norm, H, gin);
        ENG_MARK(12);
        block_sync();
        ENG_MARK(13);
        {
            const hq_layer& Ln = lay_s[final_layer ? l : l + 1];
            stage_rows<kQkvLPR, kQkvMAXC>(stage_s, !iw && !final_layer, Ln.qkv, q0, q1, H, ww);
            stage_scales<kQkvLPR>(scl_s[0], !iw && !final_layer, Ln.qkv_scales, q0, q1, ww);
        }
        act = quantize<kThreads, kActNPT>(av, I, xq_s, kDownLPR * kDownMAXC * 32, bmax);
        if (!iw && h0 + ww < h1) {
            // the staged down weights and scale, not the next layer's qkv
            // behind them (kQkvMAXC weight loads + 1 scale load)
            if (!final_layer && q0 + ww * (kWave / kQkvLPR) < q1) wait_memory_but<kQkvMAXC + 1>();
            else wait_all_memory();
            const int part = staged_dot<kDownLPR, kDownMAXC, 5>(stage_s, xq_s, ww);
            const int acc = rows_acc<kDownLPR, 0, 1>(part, lane_id());
            if (lane_id() == 0) {
                const float xn = xown_s[ww] + (float(acc) * act) * scl_s[2][ww][0];
                xown_s[ww] = xn;
                res_s[ww] = xn;
            }
        }
        block_sync();
        publish_rows(res_s, p.ll_x5 + h0, h1 - h0, E + 5);
        if (final_layer && tid < h1 - h0) p.x[h0 + tid] = res_s[tid];
        ENG_MARK(14);
        ENG_MARK(15);
    }
#ifdef HQ_ENGINE_TRACE
    block_sync();
    for (int i = tid; i < 4 * 16 * 16; i += kThreads) {
        p.trace[size_t(b) * 4 * 16 * 16 + i] = trace_s[i];
        p.trace[size_t(gridDim.x + b) * 4 * 16 * 16 + i] = atr_s[i];
        p.trace[size_t(2 * gridDim.x + b) * 4 * 16 * 16 + i] = sub_s[i];
    }
#endif
    if (b == 0 && tid == 0) *p.epoch = base + 5u * uint32_t(p.L);
}

// ---- host ---------------------------------------------------------------------

bool engine_fits(const hq_model* m)
{
    using namespace eng;
    if (m->head_dim != kD) return false;
    const int G = m->heads / m->kv_heads;
    if (G > kG || m->heads % m->kv_heads) return false;
    if (m->layers > kMaxLayers) return false;
    const int H = m->hidden, I = m->intermediate, qd = m->heads * kD;
    if (H > kMaxHidden || I > kMaxVec || qd > kMaxVec) return false;
    if (H > kIThreads * kHidNPT || qd > kIThreads * kAttNPT || I > kThreads * kActNPT) return false;
    if ((H >> 5) > kQkvLPR * kQkvMAXC || (H >> 5) > kGuLPR * 2 * kGuHalf) return false;
    if ((qd >> 5) > kOLPR * kOMAXC || (I >> 5) > kDownLPR * kDownMAXC) return false;
    return true;
}

int engine_blocks(const hq_model* m)
{
    using namespace eng;
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        int occ = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, engine_kernel, kThreads, 0) != hipSuccess ||
            occ < 1)
            n = -1;
        cus[dev] = n;
    }
    if (cus[dev] <= 0) return 0;
    const int qrows = m->heads * kD + 2 * m->kv_heads * kD;
    int nb = min(min(cus[dev], m->hidden), min(qrows, m->intermediate));
    // per-block capacities of the weight waves
    auto ceil_div = [](int a, int b) { return (a + b - 1) / b; };
    const int rpw_q = kWave / kQkvLPR;
    if (ceil_div(qrows, nb) > kWWaves * rpw_q || ceil_div(m->hidden, nb) > kWWaves ||
        ceil_div(m->hidden, nb) > kMaxOwn || ceil_div(m->intermediate, nb) > kWWaves * 4)
        return 0;
    return nb;
}

size_t engine_trace_bytes(const hq_model* m)
{
#ifdef HQ_ENGINE_TRACE
    return size_t(3 * 256) * 4 * 16 * 16 * sizeof(uint32_t);
#else
    (void)m;
    return 0;
#endif
}

size_t engine_ll_entries(const hq_model* m)
{
    const int qd = m->heads * m->head_dim;
    const int qrows = qd + 2 * m->kv_heads * m->head_dim;
    return size_t(2 * m->hidden) + size_t(qrows) + size_t(qd) + size_t(m->intermediate);
}

hipError_t launch_engine(const hq_model* m, const hq_state* st, uint64_t* ll, uint32_t* epoch,
                         float* part, int32_t* counters, int max_chunks, int nb, uint32_t* trace,
                         hipStream_t s)
{
    EngineParams p{};
    p.layers = m->device_layer;
    p.L = m->layers;
    p.H = m->hidden;
    p.I = m->intermediate;
    p.heads = m->heads;
    p.kv_heads = m->kv_heads;
    p.G = m->heads / m->kv_heads;
    const int qd = m->heads * m->head_dim;
    p.qkv_rows = qd + 2 * m->kv_heads * m->head_dim;
    p.eps = m->eps;
    p.rope_cos = m->rope_cos;
    p.rope_sin = m->rope_sin;
    p.keys = st->keys;
    p.values = st->values;
    p.kv_stride = m->kv_heads * m->head_dim;
    p.kv_layer = (long long)st->capacity * p.kv_stride;
    p.capacity = st->capacity;
    p.position = st->position;
    p.status = st->status;
    p.x = st->x;
    p.ll_x3 = ll;
    p.ll_x5 = p.ll_x3 + m->hidden;
    p.ll_qkv = p.ll_x5 + m->hidden;
    p.ll_att = p.ll_qkv + p.qkv_rows;
    p.ll_act = p.ll_att + qd;
    p.epoch = epoch;
    p.part = part;
    p.counters = counters;
    p.max_chunks = max_chunks;
    p.trace = trace;
    hipLaunchKernelGGL(engine_kernel, dim3(nb), dim3(eng::kThreads), 0, s, p);
    return hipGetLastError();
}

}  // namespace hq
