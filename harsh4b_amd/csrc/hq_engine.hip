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
// Grid: one 1024-thread block per CU, co-resident by construction (at most
// one block per CU, never more blocks than CUs).  Each block owns a slice of
// the output rows of every GEMV.  A phase's output vector is handed to every
// block as 32-bit hand-off words written with agent-scope stores and read
// with agent-scope loads until they are non-zero.  A word holds the value's
// bits XOR kHsKey, the bits of a signalling NaN, which no arithmetic result
// has, so an empty (zero) word and a published value never coincide.  Every
// layer of a launch has its own slot of words, in one of two sets
// alternating by launch: a launch clears the other set (written by the
// previous launch, which has finished) layer by layer, and the launch
// boundary makes those clears visible before the set is used again.  A
// counter in the workspace (5 epochs per layer) selects the set and tags the
// long-context attention partials, which stay 64-bit {value, epoch} entries.
//
// Wave roles (warp specialisation, no block barrier inside the layer loop):
//  * Weight waves (waves 4-15) hold their rows of the coming GEMVs in
//    registers: each GEMV's weights are loaded one to three phases ahead,
//    in the order the phases use them (vector-memory loads of one wave
//    complete in issue order, so a wave never waits for a load it does not
//    need yet).  They wait
//    for the quantized phase input in LDS, run their dot products and post
//    the results to LDS.  They issue no global stores and no polls.
//  * Input waves (waves 0-3) poll the phase inputs, run the norm and
//    quantization prologues and the attention, and publish the weight waves'
//    results.  Their global loads never queue behind weight loads of their
//    own wave.
// The two roles meet through LDS sequence counters; the four input waves
// synchronise among themselves through an LDS counter too.  Every wait on
// another block or another role is bounded: a thread whose wait spins
// kSpinLimit rounds gives up, raises HQ_STEP_SYNC in the status word and
// never waits again (`budget` becomes 0), so the kernel always finishes.
#include <utility>

#include "hq_device.h"
#include "hq_int4.h"
#include "hq_internal.h"

namespace hq {
namespace eng {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / kWave;         // 16
constexpr int kIWaves = 4;                       // input waves 0-3
constexpr int kIThreads = kIWaves * kWave;       // 256
constexpr int kWWaves = kWaves - kIWaves;        // 12 weight waves
constexpr int kD = 128;                          // head_dim
constexpr int kG = 4;                            // query heads per kv head (max)
constexpr int kMaxVec = 10240;                   // largest phase input (floats)
constexpr int kMaxHidden = 2560;
constexpr int kMaxOwn = 16;                      // residual rows per block
constexpr int kMaxRes = 64;                      // outputs of one GEMV phase per block
constexpr int kMaxLayers = 64;                   // layer table copy in LDS
constexpr int kGroup = 4;                         // chunks of 64 positions per attention item
constexpr unsigned kSpinLimit = 1u << 22;           // rounds one wait may spin
constexpr int kCopyWave0 = kIWaves, kCopyWaves = 8;  // the waves that copy attention K/V chunks into LDS
#ifdef HQ_ENGINE_TRACE
// Timestamps (low 32 bits of the 100 MHz clock) of layers kTraceL0 ..
// kTraceL0+3: input wave 0 at points 0-15, weight wave 0 at points 16-23,
// attention (input wave 0) at points 24-31.
constexpr int kTraceL0 = 16;
constexpr int kTracePoints = 96;   // 48-53: GQA item (item blocks), 54-56: GQA combine; 57-95 free
constexpr int kTraceWords = 4 * kTracePoints;
#endif

// Weight-wave layouts: LPR lanes per row, C 16-byte chunks per lane.
constexpr int kQkvLPR = 32, kQkvC = 3;           // K <= 3072, 2 rows per wave
constexpr int kOLPR = 64, kOC = 2;               // K <= 4096, 1 row per wave
constexpr int kGuLPR = 8, kGuC = 10;             // K <= 2560, 4 gate/up pairs per wave
constexpr int kDownLPR = 64, kDownC = 5;         // K <= 10240, 1 row per wave
// Phase inputs held in registers by the input threads.
constexpr int kHidNPT = kMaxHidden / kIThreads;  // 10
constexpr int kAttNPT = 16;                      // heads*D <= 4096
constexpr int kActNPT = kMaxVec / kThreads;      // 10: SwiGLU entries per thread (all waves), I <= 10240

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
    float* x;                 // residual stream: layer input in (unless token is set), final out
    // nullable: layer 0's input is row *token of the int4 embedding (the
    // step's embedding lookup, folded into the launch); x is then only written
    const int32_t* token;
    const uint8_t* emb;       // [vocab, H/2] packed int4
    const float* emb_scales;  // [vocab]
    int vocab;
    uint32_t* hs;             // hand-off words: 2 sets x L layers x hs_layer words
    int hs_layer;             // words per layer: x3 [H], x5 [H], qkv [qkv_rows], att [heads*D], act [I]
    uint32_t* epoch;
    uint64_t* ll_part;        // attention chunk partials [heads, max_chunks, D + 2] (m, l, o)
    int max_chunks;
    uint32_t* trace;          // HQ_ENGINE_TRACE builds: timestamps
};

namespace {

using namespace eng;

// f(0), f(1), ..., f(N-1) expanded at compile time (the register arrays they
// index stay in registers; a loop the optimizer declines to unroll would
// move them to scratch memory).
template <class F, int... J>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, J...>)
{
    (f(std::integral_constant<int, J>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f)
{
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// ---- LDS state shared by the roles ------------------------------------------

struct KvBuf {
    uint16_t k[kAttnChunk * kD];   // one chunk of K rows of one kv head, [t][d]
    uint16_t v[kAttnChunk * kD];
};


struct Shared {
    alignas(16) uint8_t xq[kMaxVec];    // quantized phase input, de-interleaved per 8
    float res[kMaxRes];                 // weight waves' outputs of the current phase
    float red[kIThreads];               // input-wave reductions
    float wmax[kIWaves];
    float act;                          // dequant multiplier of xq
    int xq_seq;                         // input-wave xq posts, 4 per GEMV input of P1/P3/P4 (input -> weight)
    int ibar;                           // input-wave barrier arrivals
    int hs;                             // hand-offs received by the input waves, 4 per phase
    float amx[kWaves];                  // P5: each wave's max |SwiGLU output| of its entries
    KvBuf kv[kGroup];                   // K/V chunks of the block's attention item
    alignas(16) float aq[kD];           // attention: the normalized, rotated query head
    alignas(16) float as[kGroup * kAttnChunk];   // attention: the item's scores
    alignas(16) float po[kGroup][kD];   // attention: chunk partials o, m, l
    float pm[kGroup], pl[kGroup];
    alignas(16) float gq[kG][kD];                   // GQA items: the G normalized, rotated query heads
    alignas(16) float gs[kG][kGroup * kAttnChunk];  // GQA items: their scores
    hq_layer lay[kMaxLayers];
#ifdef HQ_ENGINE_TRACE
    uint32_t trace[kTraceWords];
#endif
};

// The kernel's LDS, at namespace scope so every helper addresses it as LDS
// (32-bit offsets) rather than through generic pointers.
__shared__ Shared S;


// The thread index, opaque to the optimizer: addresses derived from it
// inside the layer loops are loop-invariant, and hoisting all of them out of
// a loop holds more registers than the loop body itself needs.
__device__ __forceinline__ int opaque_tid()
{
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}
__device__ __forceinline__ int lane_id() { return opaque_tid() & (kWave - 1); }

__device__ __forceinline__ int lds_load(const int* p)
{
    return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// The wave's LDS operations have completed (issued in order, so a flag
// written after this is seen after the data written before it).
__device__ __forceinline__ void lds_drain() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

__device__ __forceinline__ float lane_f(float v, int lane)
{
    return bits_f32(__builtin_amdgcn_readlane(f32_bits(v), lane));
}

// Block barrier for LDS data: this wave's LDS operations complete, then
// s_barrier.  Unlike __syncthreads it does not wait for the wave's global
// memory operations, so weight loads in flight stay in flight.  The weight
// waves hand each GEMV's results to the input waves through it (the input
// waves are idle then, and the barrier releases them sooner than a polled
// LDS count: 36 layers at context 64 went from 810 to 750 us per launch).
// The input waves hand the quantized phase input on through the xq_seq count
// instead: as a barrier it would hold their prologue until the weight waves
// had issued their next loads (765 us).
__device__ __forceinline__ void block_sync()
{
    lds_drain();
    __builtin_amdgcn_s_barrier();
    compiler_fence();
}

// Wait until *p >= target (LDS), bounded.
__device__ __forceinline__ void wait_lds_geq(const int* p, int target, unsigned& budget, int32_t* status)
{
    unsigned spins = 0;
    while (lds_load(p) < target && budget != 0) {
        __builtin_amdgcn_s_sleep(1);
        if (++spins == kSpinLimit) { budget = 0; atomicOr(status, HQ_STEP_SYNC); }
    }
    compiler_fence();
}

// Barrier of the four input waves (every input thread calls it with the same
// running count `seq`).
__device__ __forceinline__ void ibar(int& seq, unsigned& budget, int32_t* status)
{
    seq += kIWaves;
    lds_drain();
    if (lane_id() == 0) __hip_atomic_fetch_add(&S.ibar, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    // (spun without s_sleep: the four input waves arrive within a few
    // hundred clocks of each other)
    unsigned spins = 0;
    while (lds_load(&S.ibar) < seq && budget != 0)
        if (++spins == kSpinLimit) { budget = 0; atomicOr(status, HQ_STEP_SYNC); }
}

#ifdef HQ_ENGINE_TRACE
#define TRACE(l, point)                                                                          \
    do {                                                                                         \
        if ((l) >= kTraceL0 && (l) < kTraceL0 + 4)                                               \
            S.trace[((l) - kTraceL0) * kTracePoints + (point)] = uint32_t(wall_clock64());       \
    } while (0)
#else
#define TRACE(l, point) do { } while (0)
#endif

// ---- global hand-off words ------------------------------------------------------

constexpr uint32_t kHsKey = 0x7FA5A5A5u;   // a signalling-NaN pattern (quiet bit clear)

__device__ __forceinline__ void hs_store(uint32_t* p, float v)
{
    __hip_atomic_store(p, f32_bits(v) ^ kHsKey, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool hs_ready(uint32_t w) { return w != 0u; }
__device__ __forceinline__ float hs_value(uint32_t w) { return bits_f32(w ^ kHsKey); }

// One layer's slot of hand-off words in the launch's set: x3 [H], x5 [H],
// qkv [qkv_rows], att [heads*D], act [I].  Only the slot base is carried;
// the vector addresses are recomputed where they are used (a few scalar
// instructions), which holds fewer registers across the layer loop.
struct Slot {
    uint32_t* base;
    int H, qkv_rows, qd;
    __device__ __forceinline__ uint32_t* x3() const { return base; }
    __device__ __forceinline__ uint32_t* x5() const { return base + H; }
    __device__ __forceinline__ uint32_t* qkv() const { return base + 2 * H; }
    __device__ __forceinline__ uint32_t* att() const { return base + 2 * H + qkv_rows; }
    __device__ __forceinline__ uint32_t* act() const { return base + 2 * H + qkv_rows + qd; }
};
__device__ __forceinline__ Slot slot_of(const EngineParams& p, int set, int l)
{
    return Slot{p.hs + (size_t(set) * size_t(p.L) + size_t(l)) * size_t(p.hs_layer), p.H, p.qkv_rows,
                p.heads * 128};
}

// ---- 64-bit {value, epoch} entries (attention chunk partials) -------------------

__device__ __forceinline__ void ll_store(uint64_t* p, float v, uint32_t epoch)
{
    __hip_atomic_store(p, (uint64_t(epoch) << 32) | uint64_t(f32_bits(v)), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
// Hand-off vectors are read through scalar buffer descriptors: a load takes
// one 32-bit lane offset plus a scalar offset, so the polls of a phase hold
// no 64-bit address registers.  sc1 makes the load coherent at agent scope
// (the same instruction as an agent-scope atomic load); spin loops re-read
// after a compiler memory fence, so no read is merged with an earlier one.
constexpr int kBufSC1 = 16;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, int bytes = 0x7fffffff)
{
    // gfx9 raw buffer: stride 0; loads at or past `bytes` return 0 and touch
    // no memory
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(uniform_ptr(p)), 0,
                                             __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}
__device__ __forceinline__ bool ll_ready(uint64_t v, uint32_t epoch)
{
    return int32_t(uint32_t(v >> 32) - epoch) >= 0;
}
__device__ __forceinline__ uint32_t hs_load(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff)
{
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, kBufSC1);
}

__device__ __forceinline__ int split_begin(int n, int b, int nb) { return int((long long)n * b / nb); }

// Pointers read from the device layer table are generic to the compiler;
// reading through a global-address-space pointer gives global (not flat)
// loads.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gmem(const T* p)
{
    return (const __attribute__((address_space(1))) T*)p;
}

// Lane 0 of the calling wave waits until the last entry of src[0, n) is
// current; the wave then reads its part of the vector in one burst
// (poll_into re-reads the few entries that are not current yet).  Every
// block polls the same entry, so the wait costs a load per watching wave
// and round: the polls of the 256 blocks share the memory channels with the
// producers' stores, and few watchers measured faster hand-offs (64
// watching lanes per block 929 us per launch of all 36 layers, 16 lanes 899
// us, 4 lanes 877 us, 1 lane 861 us, in a build where the other input waves
// then met wave 0 at a barrier).  Each input wave watches for itself: that
// costs fewer than the barrier after one wave's watch (746 -> 739 us).
__device__ __forceinline__ void watch_last(const uint32_t* src, int n, unsigned& budget, int32_t* status)
{
    if (lane_id() == 0 && n > 0) {
        const __amdgpu_buffer_rsrc_t r = buffer_rsrc(src);
        const uint32_t off = uint32_t(n - 1) * 4u;
        uint32_t w = hs_load(r, off, 0);
        unsigned spins = 0;
        while (!hs_ready(w) && budget != 0) {
            __builtin_amdgcn_s_sleep(1);
            if (++spins == kSpinLimit) { budget = 0; atomicOr(status, HQ_STEP_SYNC); }
            compiler_fence();
            w = hs_load(r, off, 0);
        }
    }
}

// Hand-off words: thread t polls words t, t+STRIDE, ... of src[0, n) until
// they are non-zero and returns their values in out[] (0.0f past n).  All
// loads are in flight at once; while waiting, a thread re-reads the words
// that are still empty (the caller has watched the vector's last word first,
// so the burst rarely needs a second round).
template <int NPT, int STRIDE = kIThreads>
__device__ __forceinline__ void poll_into(const uint32_t* src, int n, float (&out)[NPT], unsigned& budget,
                                          int32_t* status)
{
    const int t = opaque_tid();
    const __amdgpu_buffer_rsrc_t r = buffer_rsrc(src, n * 4);   // words past n read as 0
    const uint32_t vo = uint32_t(t) * 4u;
    uint32_t v[NPT];
    static_for<NPT>([&](auto j) { v[j] = hs_load(r, vo, j * STRIDE * 4); });
    unsigned spins = 0;
    while (budget != 0) {
        uint64_t pending = 0;
        static_for<NPT>([&](auto j) {
            pending |= uint64_t(int(t + STRIDE * j < n) & int(!hs_ready(v[j]))) << j;
        });
        if (pending == 0) break;
        __builtin_amdgcn_s_sleep(1);
        if (++spins == kSpinLimit) { budget = 0; atomicOr(status, HQ_STEP_SYNC); }
        compiler_fence();
        static_for<NPT>([&](auto j) {
            if ((pending >> j) & 1) v[j] = hs_load(r, vo, j * STRIDE * 4);
        });
    }
    static_for<NPT>([&](auto j) { out[j] = t + STRIDE * j < n ? hs_value(v[j]) : 0.0f; });
}

// ---- input-wave prologues ---------------------------------------------------------
//
// The phase input is held in registers, element t + 256*j in x[j] of input
// thread t, 0 past n.  The int8 result goes to S.xq in the de-interleaved
// layout, zero-padded up to npad (the GEMV layouts read whole chunk spans:
// a zero activation makes a padded chunk contribute 0).

// Max over the four input waves (order-free).
__device__ __forceinline__ float inputs_max(float v, int& bseq, unsigned& budget, int32_t* status)
{
    v = wave_max64_all(v);
    if (lane_id() == 0) S.wmax[opaque_tid() / kWave] = v;
    ibar(bseq, budget, status);
    return fmaxf(fmaxf(S.wmax[0], S.wmax[1]), fmaxf(S.wmax[2], S.wmax[3]));
}

template <int NPT>
__device__ __forceinline__ void write_xq(const float (&x)[NPT], float inv, int n, int npad)
{
    static_assert(kIThreads * NPT <= kMaxVec, "xq stores past the buffer");
    const int t = opaque_tid();
#pragma unroll
    for (int j = 0; j < NPT; ++j) S.xq[xq_offset(t + kIThreads * j)] = uint8_t(quant_i8(x[j], inv));
    for (int i = max(n, kIThreads * NPT) + t; i < npad; i += kIThreads) S.xq[i] = 0;
}

// RMSNorm (the spec's 256 strided fmaf partials, halving tree) then
// quantization of this wave's elements into S.xq; returns the dequant
// multiplier (post_xq hands the result on).
template <int NPT>
__device__ __forceinline__ float rmsnorm_quant(float (&x)[NPT], int n, const float (&gam)[NPT],
                                               float eps, int npad, int& bseq, unsigned& budget, int32_t* status,
                                               int tl = -1, int tp = 0)
{
    const int t = opaque_tid();
    n = __builtin_amdgcn_readfirstlane(n);   // (uniform; an SGPR operand for the asm below)
    asm volatile("" : "+s"(n));   // keep float(n) from being hoisted out of the layer loop
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NPT; ++j) ss = __builtin_fmaf(x[j], x[j], ss);
    S.red[t] = ss;
    TRACE(tl, tp);
    ibar(bseq, budget, status);
    TRACE(tl, tp + 1);
    // levels 128 and 64 of the tree (partial i + partial i + o), then the
    // wave tree over the 64 remaining partials; every wave computes the same
    // total from the same LDS values
    const int l = lane_id();
    const float r2 = (S.red[l] + S.red[l + 128]) + (S.red[l + 64] + S.red[l + 192]);
    const float total = wave_tree_sum64_all(r2);
    const float r = __builtin_sqrtf(total / float(n) + eps);
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < NPT; ++j) x[j] = (x[j] / r) * gam[j];
#pragma unroll
    for (int j = 0; j < NPT; ++j) amax = fmaxf(amax, fabsf(x[j]));
    TRACE(tl, tp + 2);
    amax = fmaxf(inputs_max(amax, bseq, budget, status), 1e-5f);
    TRACE(tl, tp + 3);
    write_xq(x, 127.0f / amax, n, npad);
    TRACE(tl, tp + 4);
    return amax / 127.0f;
}

template <int NPT>
__device__ __forceinline__ float quantize(const float (&x)[NPT], int n, int npad, int& bseq,
                                          unsigned& budget, int32_t* status)
{
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < NPT; ++j) amax = fmaxf(amax, fabsf(x[j]));
    amax = fmaxf(inputs_max(amax, bseq, budget, status), 1e-5f);
    write_xq(x, 127.0f / amax, n, npad);
    return amax / 127.0f;
}

// Hand this wave's part of the phase input to the weight waves: its xq
// writes and the (same in every input wave) dequant multiplier are complete
// before its count; the weight waves wait for all four counts of a phase.
__device__ __forceinline__ void post_xq(float act)
{
    if (lane_id() == 0) S.act = act;
    lds_drain();
    if (lane_id() == 0) __hip_atomic_fetch_add(&S.xq_seq, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// This input wave has received a phase's hand-off: the weight waves time
// their next loads by it.
__device__ __forceinline__ void post_hs()
{
    if (lane_id() == 0) __hip_atomic_fetch_add(&S.hs, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

template <int NPT>
__device__ __forceinline__ void load_gamma(const float* g, int n, float (&out)[NPT])
{
    const int t = opaque_tid();
    const __amdgpu_buffer_rsrc_t r = buffer_rsrc(g, n * 4);   // elements past n read as 0
    static_for<NPT>([&](auto j) {
        out[j] = bits_f32(__builtin_amdgcn_raw_buffer_load_b32(r, uint32_t(t) * 4u, j * kIThreads * 4, 0));
    });
}

// ---- P5 input, all sixteen waves ------------------------------------------------------
//
// The SwiGLU output arrives as fp32 hand-off entries (every block's rows).
// One lane watches the last of them; then every thread T of the
// block reads entries T, T+1024, ..., the waves agree on the maximum |value|
// through LDS, and each thread quantizes its own entries into S.xq.  The
// weight waves hold only the down rows at this point (their loads have long
// landed), so their polls do not queue behind weight loads.  Returns the
// dequant multiplier amax/127 (the same in every wave).
__device__ float act_phase(const EngineParams& p, int l, const uint32_t* act, unsigned& budget)
{
    const int T = opaque_tid();
    const int w = T / kWave;
    const int I = p.I;
    // Every wave of the block calls this once per layer, so the block
    // barriers below match up across the two roles.
    if (w == 0) watch_last(act, I, budget, p.status);
    __syncthreads();
    if (w == 0) TRACE(l, 12);
    if (w == kIWaves) TRACE(l, 15);
    float a[kActNPT];
    poll_into<kActNPT, kThreads>(act, I, a, budget, p.status);
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < kActNPT; ++j) m = fmaxf(m, fabsf(a[j]));   // 0 past I
    m = wave_max64_all(m);
    if (lane_id() == 0) S.amx[w] = m;
    block_sync();
    if (w == 0) TRACE(l, 42);
    if (w == kIWaves) TRACE(l, 30);
    // the sixteen wave maxima in lanes 0-15 of each row, folded by the row's
    // DPP shifts into its lane 0 (maxima of non-negative values: order-free)
    static_assert(kWaves == 16, "one wave maximum per row lane");
    float amax = S.amx[lane_id() & 15];
    amax = fmaxf(amax, dpp_f<kRowShl8>(amax));
    amax = fmaxf(amax, dpp_f<kRowShl4>(amax));
    amax = fmaxf(amax, dpp_f<kRowShl2>(amax));
    amax = fmaxf(amax, dpp_f<kRowShl1>(amax));
    amax = fmaxf(lane_f(amax, 0), 1e-5f);
    const float inv = 127.0f / amax;
    // every element of the down GEMV's span, I included: a[j] is 0 past I,
    // which quantizes to the zero padding
    static_assert(kActNPT * kThreads == kDownLPR * kDownC * 32, "quantized span = the down rows' span");
#pragma unroll
    for (int j = 0; j < kActNPT; ++j) S.xq[xq_offset(T + kThreads * j)] = uint8_t(quant_i8(a[j], inv));
    block_sync();
    if (w == 0) TRACE(l, 44);
    if (w == kIWaves) TRACE(l, 31);
    return amax / 127.0f;
}

// ---- weight waves ---------------------------------------------------------------
//
// Weights are read with buffer loads: the matrix base is a scalar buffer
// descriptor and each load takes one 32-bit lane offset, so the loads of a
// phase hold no 64-bit address registers.  Cache policy: non-temporal (the
// weights are read once per step).
constexpr int kBufNT = 2;

// Weight-load pacing: a weight wave waits WAVE_GAP (s_sleep units of 64
// clocks) per wave index before a phase's loads and CHUNK_GAP between its
// chunk loads, so the next phase's weights stream in over a few
// microseconds instead of one burst that would queue ahead of the
// hand-off reads in the memory system.
constexpr int pace(int wave_gap, int chunk_gap) { return wave_gap << 8 | chunk_gap; }
constexpr int kPaceQkv = pace(0, 0), kPaceO = pace(0, 0), kPaceGu = pace(0, 0), kPaceDown = pace(0, 0);

template <int P>
__device__ __forceinline__ void pace_start(int ww)
{
    if constexpr ((P >> 8) > 0)
        for (int i = 0; i < ww; ++i) __builtin_amdgcn_s_sleep(P >> 8);
}
template <int P>
__device__ __forceinline__ void pace_chunk(int j)
{
    if constexpr ((P & 255) > 0)
        if (j > 0) __builtin_amdgcn_s_sleep(P & 255);
}

__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kBufNT);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Rows [r0, r1) of a GEMV; weight wave ww owns RPW = 64/LPR consecutive rows
// from r0 + ww*RPW (clamped to r1 - 1), lane li = lane % LPR of a row reads
// chunks li + j*LPR (clamped into the row: a clamped chunk meets zero
// activations).  Each lane also loads the scale of its own row.  A wave
// without rows loads the block's last row and discards it (a conditional
// load would keep the registers' previous contents alive across the loop).
template <int LPR, int C, int P>
__device__ __forceinline__ void load_rows(uint4 (&w)[C], float& s, const uint8_t* W, const float* Sc, int r0,
                                          int r1, int K, int ww)
{
    constexpr int RPW = kWave / LPR;
    const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(W);
    const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(Sc);
    const int lane = lane_id();
    const int row = min(r0 + ww * RPW + lane / LPR, r1 - 1);
    const int li = lane % LPR;
    const int nch = K >> 5;
    const uint32_t off = uint32_t(row) * uint32_t(K >> 1);
    pace_start<P>(ww);
    s = bits_f32(__builtin_amdgcn_raw_buffer_load_b32(rs, uint32_t(row) * 4u, 0, 0));
#pragma unroll
    for (int j = 0; j < C; ++j) {
        pace_chunk<P>(j);
        w[j] = bload16(rw, off + uint32_t(min(li + j * LPR, nch - 1)) * 16u);
    }
}

// SwiGLU rows: pairs [p0, p1) of the I gate rows; weight wave ww owns pairs
// p0 + 4*ww .. +3, lane groups 0-3 read the gate rows and 4-7 the matching
// up rows (row I + pair); chunks li + j*8.
// Chunks [J0, J1) of the wave's pairs (the scale with the first part).
template <int J0, int J1>
__device__ __forceinline__ void load_pairs(uint4 (&w)[kGuC], float& s, const uint8_t* W, const float* Sc, int p0,
                                           int p1, int I, int K, int ww)
{
    const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(W);
    const int lane = lane_id();
    const int rsel = lane >> 3;
    const int pair = min(p0 + ww * 4 + (rsel & 3), p1 - 1);
    const int row = rsel < 4 ? pair : I + pair;
    const int li = lane & 7;
    const int nch = K >> 5;
    const uint32_t off = uint32_t(row) * uint32_t(K >> 1);
    if constexpr (J0 == 0) {
        const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(Sc);
        pace_start<kPaceGu>(ww);
        s = bits_f32(__builtin_amdgcn_raw_buffer_load_b32(rs, uint32_t(row) * 4u, 0, 0));
    }
#pragma unroll
    for (int j = J0; j < J1; ++j) {
        pace_chunk<kPaceGu>(j);
        w[j] = bload16(rw, off + uint32_t(min(li + j * 8, nch - 1)) * 16u);
    }
}

// 16 * partial dot product of this lane's C chunks with the LDS activations.
template <int LPR, int C>
__device__ __forceinline__ int reg_dot(const uint4 (&w)[C], const uint8_t* xq)
{
    const int li = lane_id() % LPR;
    int a0 = 0, a1 = 0, a2 = 0, a3 = 0;
#pragma unroll
    for (int j = 0; j < C; j += 2) {
        dot_chunk(w[j], xq + (li + j * LPR) * 32, a0, a1);
        if (j + 1 < C) dot_chunk(w[j + 1], xq + (li + (j + 1) * LPR) * 32, a2, a3);
        // two chunks' activations in flight at a time: hoisting all of them
        // would need more registers than the wave holds
        __builtin_amdgcn_sched_barrier(0);
    }
    return (a0 + a1) + (a2 + a3);
}

// Lane r < COUNT receives the accumulator of the wave's row FIRST + r.
template <int LPR, int FIRST, int COUNT>
__device__ __forceinline__ int rows_acc(int part)
{
    static_assert(FIRST + COUNT <= kWave / LPR, "row outside the wave");
    const int lane = lane_id();
    int acc = 0;
#pragma unroll
    for (int r = 0; r < COUNT; ++r) {
        const int t = row_isum<LPR>(part, FIRST + r) >> 4;
        if (lane == r) acc = t;
    }
    return acc;
}



struct Rows {
    int h0, h1, q0, q1, g0, g1;
};

// Weight loads are issued once the input waves have received hand-off e
// (4 per layer: inputs of qkv, o, gate_up and down): the weights then stream
// while the input waves compute, not while the next hand-off is in flight.
constexpr bool kLoadInWindows = true;

__device__ __forceinline__ void load_window(int e, unsigned& budget, int32_t* status)
{
    if constexpr (kLoadInWindows) wait_lds_geq(&S.hs, kIWaves * (e + 1), budget, status);
}

__device__ void attention_phase(const EngineParams& p, const hq_layer& Ly, int l, int pos, const Slot& z,
                                uint32_t epoch_att, unsigned& budget);
__device__ __forceinline__ bool is_copy_wave(int w);
template <bool GQA>
__device__ __forceinline__ void prefetch_first_item(const EngineParams& p, int l, int pos);

__device__ __forceinline__ bool block_has_item(const EngineParams& p, int pos);

// (Both roles are forced inline: compiled out of line, as the traced build's
// larger code was, the role function took the kernel parameters through
// scratch memory and spilled, and its timestamps no longer showed the
// untraced kernel's timing.)
__device__ __forceinline__ void weight_role(const EngineParams& p, const Rows& R, int ww, int pos, uint32_t base,
                                            int set, unsigned& budget)
{
    const int H = p.H, I = p.I;
    const int qd = p.heads * kD;
    const int lane = lane_id();
    // every wave runs every dot (a wave without rows of a GEMV computes on
    // the clamped last row and stores nothing), so each dot waits for exactly
    // its own weight loads on every path
    const bool has_o = R.h0 + ww < R.h1;
    // Loads are issued in the order the phases use them, each after the dot
    // that frees its registers and, mostly, once the input waves hold the
    // next hand-off: gate_up after the attention phase, down once the
    // attention residual is in, the next layer's qkv once the down input is
    // in and its o once the layer output is in.  Every GEMV's weights so
    // have one to two hand-offs of lead time while a wave holds at most
    // about two phases of weights.  A block without attention items issues
    // its gate_up loads as soon as it leaves the attention phase: they land
    // while the attention runs elsewhere, and none is in flight when the
    // attention residual's hand-off is read (a wave's memory operations
    // complete in issue order, so loads issued ahead of a hand-off read
    // delay it).  Blocks with items wait for the attention output first.
    // (36 layers at context 64: 835 us per launch against 841 with every
    // block loading three chunks after the attention output and seven after
    // its o dot; 987 against 1012 us at context 1024.)
    uint4 wq[kQkvC] = {}, wo[kOC] = {}, wg[kGuC] = {}, wd[kDownC] = {};
    const bool att_blk = block_has_item(p, pos);
    float sq = 0.0f, so = 0.0f, sg = 0.0f, sd = 0.0f;
    load_rows<kQkvLPR, kQkvC, pace(0, 0)>(wq, sq, S.lay[0].qkv, S.lay[0].qkv_scales, R.q0, R.q1, H, ww);
    load_rows<kOLPR, kOC, pace(0, 0)>(wo, so, S.lay[0].o, S.lay[0].o_scales, R.h0, R.h1, qd, ww);
#pragma unroll 1
    for (int l = 0; l < p.L; ++l) {
        const bool more = l + 1 < p.L;
        const hq_layer& Ly = S.lay[l];
        const hq_layer& Ln = S.lay[more ? l + 1 : l];
        // the first layer's first attention item (GQA or per head): its K/V
        // copies land while the qkv GEMV and its hand-off run (later layers
        // issue theirs at the end of the layer before)
        if (l == 0 && is_copy_wave(opaque_tid() / kWave)) {
            prefetch_first_item<true>(p, l, pos);
            prefetch_first_item<false>(p, l, pos);
        }
        // ---- P1: qkv
        wait_lds_geq(&S.xq_seq, kIWaves * (3 * l + 1), budget, p.status);
        if (ww == 0) TRACE(l, 16);
        {
            const float act = S.act;
            const int acc = rows_acc<kQkvLPR, 0, 2>(reg_dot<kQkvLPR, kQkvC>(wq, S.xq));
            const int row = R.q0 + ww * 2 + lane;
            const float sc = lane == 0 ? lane_f(sq, 0) : lane_f(sq, kQkvLPR);
            if (lane < 2 && row < R.q1) S.res[row - R.q0] = (float(acc) * act) * sc;
        }
        block_sync();   // results in S.res
        if (ww == 0) TRACE(l, 17);
        if (ww == kWWaves - 1) TRACE(l, 47);
        // ---- P2: the block's attention items (all waves)
        attention_phase(p, Ly, l, pos, slot_of(p, set, l), base + 5u * uint32_t(l) + 2u, budget);
        if (att_blk) load_window(4 * l + 1, budget, p.status);
        load_pairs<0, kGuC>(wg, sg, Ly.gate_up, Ly.gate_up_scales, R.g0, R.g1, I, H, ww);
        // ---- P3: o (the residual add is the input waves')
        wait_lds_geq(&S.xq_seq, kIWaves * (3 * l + 2), budget, p.status);
        if (ww == 0) TRACE(l, 18);
        if (ww == kWWaves - 1) TRACE(l, 45);
        {
            const float act = S.act;
            const int acc = rows_acc<kOLPR, 0, 1>(reg_dot<kOLPR, kOC>(wo, S.xq));
            if (has_o && lane == 0) S.res[ww] = (float(acc) * act) * so;
        }
        block_sync();   // results in S.res
        if (ww == 0) TRACE(l, 19);
        if (ww == kWWaves - 1) TRACE(l, 46);
        load_window(4 * l + 2, budget, p.status);
        load_rows<kDownLPR, kDownC, kPaceDown>(wd, sd, Ly.down, Ly.down_scales, R.h0, R.h1, I, ww);
        // ---- P4: gate_up + SwiGLU
        wait_lds_geq(&S.xq_seq, kIWaves * (3 * l + 3), budget, p.status);
        if (ww == 0) TRACE(l, 20);
        {
            const float act = S.act;
            const int part = reg_dot<kGuLPR, kGuC>(wg, S.xq);
            const int acc = rows_acc<kGuLPR, 0, 4>(part);
            const int acc_up = rows_acc<kGuLPR, 4, 4>(part);
            const int pair = R.g0 + ww * 4 + lane;
            float sgl = lane_f(sg, 0), sul = lane_f(sg, 32);
            sgl = lane == 1 ? lane_f(sg, 8) : sgl;
            sul = lane == 1 ? lane_f(sg, 40) : sul;
            sgl = lane == 2 ? lane_f(sg, 16) : sgl;
            sul = lane == 2 ? lane_f(sg, 48) : sul;
            sgl = lane == 3 ? lane_f(sg, 24) : sgl;
            sul = lane == 3 ? lane_f(sg, 56) : sul;
            if (lane < 4 && pair < R.g1) {
                const float g = (float(acc) * act) * sgl;
                const float u = (float(acc_up) * act) * sul;
                const float t = 1.0f + spec_expf(-g);
                S.res[pair - R.g0] = (g / t) * u;
            }
        }
        block_sync();   // results in S.res
        if (ww == 0) TRACE(l, 21);
        // (after the last layer the same loads, all of one 16-byte block:
        // the instruction sequence, and so every dot's wait, is the same on
        // every path)
        // ---- P5: down (the residual add is the input waves')
        const float act5 = act_phase(p, l, slot_of(p, set, l).act(), budget);
        load_rows<kQkvLPR, kQkvC, kPaceQkv>(wq, sq, Ln.qkv, Ln.qkv_scales, R.q0, more ? R.q1 : R.q0 + 1,
                                            more ? H : 32, ww);
        if (ww == 0) TRACE(l, 22);
        {
            const float act = act5;
            const int acc = rows_acc<kDownLPR, 0, 1>(reg_dot<kDownLPR, kDownC>(wd, S.xq));
            if (has_o && lane == 0) S.res[ww] = (float(acc) * act) * sd;
        }
        block_sync();   // results in S.res
        if (ww == 0) TRACE(l, 23);
        // the next layer's first attention item (GQA or per head): its K/V
        // copies (cached positions only; the current position's row comes
        // from the qkv hand-off) are issued now, while the layer's own
        // attention and its combine staging are done with S.kv.  The next
        // wait that covers them (memory operations complete in issue order)
        // is the next layer's qkv dot, a residual hand-off and an RMSNorm
        // prologue later.  (Per-head items' copies issued after the qkv dot
        // instead held the item block's polls of the qkv rows behind them:
        // 36 layers 711.5 -> 706.5 us per launch at context 70, 739.5 ->
        // 721.7 at 136, 801.5 -> 742.2 at 256.)
        if (more && is_copy_wave(opaque_tid() / kWave)) {
            prefetch_first_item<true>(p, l + 1, pos);
            prefetch_first_item<false>(p, l + 1, pos);
        }
        if (more) load_window(4 * (l + 1), budget, p.status);
        load_rows<kOLPR, kOC, kPaceO>(wo, so, Ln.o, Ln.o_scales, R.h0, more ? R.h1 : R.h0 + 1, more ? qd : 32, ww);
    }
}

// ---- attention (P2) ----------------------------------------------------------------
//
// Work item = (kv head, chunk of 64 positions), one block per item, its
// four input waves = the query heads of the kv head (same arithmetic as
// attention_kernel's STEP mode in hq_attention.hip).  The chunk's K and V
// rows are copied from HBM into LDS with gfx950's global->LDS loads before
// the qkv hand-off is awaited, so they arrive while it travels.

// Copies K and V rows [t0, t0 + 64) of kv head kvh into S.kv[kb]: rows
// before the current position from the cache, rows after it as zeros; the
// row of the current position is written from the qkv hand-off.  The copies
// are issued by the kCopyWaves copy waves (weight waves 4..11, idle during
// attention), each handling 8 rows of K and of V: one instruction moves 4
// rows of 128 halves.  A wave's loads complete in issue order, so copies
// issued by the input waves would hold back their next hand-off polls.
__device__ __forceinline__ bool is_copy_wave(int w) { return w >= kCopyWave0 && w < kCopyWave0 + kCopyWaves; }

__device__ __forceinline__ void prefetch_kv(const EngineParams& p, int l, int kvh, int t0, int n, int pos, int kb)
{
    const int w = opaque_tid() / kWave - kCopyWave0;
    const int lane = lane_id();
    const uint16_t* kl = p.keys + size_t(l) * size_t(p.kv_layer);
    const uint16_t* vl = p.values + size_t(l) * size_t(p.kv_layer);
    const uint32_t kdst = lds_addr(S.kv[kb].k), vdst = lds_addr(S.kv[kb].v);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = w * 8 + i * 4 + (lane >> 4);             // row within the chunk
        const int t = t0 + r;
        const uint32_t off = uint32_t((size_t(min(t, n - 1)) * size_t(p.kv_stride) + size_t(kvh) * kD +
                                       size_t(lane & 15) * 8) * 2);
        const uint32_t row0 = uint32_t((w * 8 + i * 4) * kD * 2);
        if (t < pos) {
            dma16(kl, off, kdst + row0);
            dma16(vl, off, vdst + row0);
        } else if (t > pos) {
            // past the context: zeros, so the V accumulation may run over
            // the whole chunk (e_t = 0 there) without branches
            *reinterpret_cast<uint4*>(&S.kv[kb].k[r * kD + (lane & 15) * 8]) = make_uint4(0, 0, 0, 0);
            *reinterpret_cast<uint4*>(&S.kv[kb].v[r * kD + (lane & 15) * 8]) = make_uint4(0, 0, 0, 0);
        }
    }
}

// K/V of chunks c0 .. c0+ncg-1 of kv head kvh into S.kv[0 .. ncg) (copy waves).
__device__ __forceinline__ void prefetch_group(const EngineParams& p, int l, int kvh, int c0, int ncg, int n,
                                               int pos)
{
    for (int c = 0; c < ncg; ++c) prefetch_kv(p, l, kvh, (c0 + c) * kAttnChunk, n, pos, c);
}

__device__ __forceinline__ int gqa_group(int nc, int kv_heads, int nb);
__device__ __forceinline__ int item_slot(int b, int NB, int G);

// The copies of this block's first attention item of layer l (copy waves),
// GQA items (GQA true: more than kGroup chunks, up to three per item) and
// per-head items (GQA false) alike: issued at the end of layer l - 1 (layer
// 0: at its start), so they land while the qkv GEMV and its hand-off run
// and none is still queued when the item polls for its qkv rows.
// Items as in attention_phase.
template <bool GQA>
__device__ __forceinline__ void prefetch_first_item(const EngineParams& p, int l, int pos)
{
    const int n = pos + 1;
    const int nc = (n + kAttnChunk - 1) / kAttnChunk;
    const int ng = (nc + kGroup - 1) / kGroup;
    const int b = blockIdx.x;
    if (GQA && ng > 1) {
        const int cg = gqa_group(nc, p.kv_heads, gridDim.x);
        const int ngq = (nc + cg - 1) / cg;
        if (b < p.kv_heads * ngq) prefetch_group(p, l, b / ngq, (b % ngq) * cg, min(cg, nc - (b % ngq) * cg), n, pos);
    } else if (!GQA && ng == 1) {
        const int k = item_slot(b, gridDim.x, p.G);   // per-head item: query head k
        if (k < p.heads) prefetch_group(p, l, k / p.G, 0, nc, n, pos);
    }
}

// Whether this block runs an attention item of every layer at position pos
// (the item assignment of attention_phase).
__device__ __forceinline__ bool block_has_item(const EngineParams& p, int pos)
{
    const int n = pos + 1;
    const int nc = (n + kAttnChunk - 1) / kAttnChunk;
    if ((nc + kGroup - 1) / kGroup > 1) {
        const int cg = gqa_group(nc, p.kv_heads, gridDim.x);
        return int(blockIdx.x) < p.kv_heads * ((nc + cg - 1) / cg);
    }
    return item_slot(blockIdx.x, gridDim.x, p.G) < p.heads;
}

// n when the blocks that run attention items at position pos are exactly
// blocks [0, n) (as block_has_item assigns them), else -1.
__device__ __forceinline__ int item_block_prefix(const EngineParams& p, int pos)
{
    const int n = pos + 1;
    const int nc = (n + kAttnChunk - 1) / kAttnChunk;
    const int NB = int(gridDim.x);
    if ((nc + kGroup - 1) / kGroup > 1) {
        const int cg = gqa_group(nc, p.kv_heads, NB);
        return min(NB, p.kv_heads * ((nc + cg - 1) / cg));
    }
    // item_slot maps blocks [0, 32k) onto slots [0, 32k), else it is the identity
    if (p.G != 4 || (NB & 31) != 0 || (p.heads & 31) == 0) return min(NB, p.heads);
    return -1;
}

// V accumulation of one or two chains per lane: o[d] = fmaf chain of
// e_t * v_t[d] over ascending t of a chunk (positions past the context have
// e_t = 0 and zero V rows: their fmaf returns the accumulator unchanged, bit
// for bit).  V values are read eight positions ahead of the chain.
template <int NCH>
__device__ __forceinline__ void v_chains(const uint16_t* va, const uint16_t* vb, float ea, float eb, float& oa,
                                         float& ob)
{
    constexpr int kB = 8 / NCH;
    uint16_t xa[2][kB], xb[2][kB];
    static_for<kB>([&](auto j) {
        xa[0][j] = va[j * kD];
        if constexpr (NCH == 2) xb[0][j] = vb[j * kD];
    });
    static_for<kAttnChunk / kB>([&](auto bt) {
        constexpr int t0 = bt * kB;
        constexpr int cur = bt & 1;
        if constexpr (t0 + kB < kAttnChunk)
            static_for<kB>([&](auto j) {
                xa[cur ^ 1][j] = va[(t0 + kB + j) * kD];
                if constexpr (NCH == 2) xb[cur ^ 1][j] = vb[(t0 + kB + j) * kD];
            });
        __builtin_amdgcn_sched_barrier(0);
        static_for<kB>([&](auto j) {
            oa = __builtin_fmaf(lane_f(ea, t0 + j), f16_to_f32(xa[cur][j]), oa);
            if constexpr (NCH == 2) ob = __builtin_fmaf(lane_f(eb, t0 + j), f16_to_f32(xb[cur][j]), ob);
        });
    });
}

// Softmax terms of chunk c of the item (scores in S.as): the chunk maximum,
// e_t in lane t, and the tree sum of the e_t.
__device__ __forceinline__ void chunk_softmax(int c, int tn, float& m, float& ex, float& ls)
{
    const int lane = lane_id();
    const float sc = S.as[c * kAttnChunk + lane];
    m = wave_max64_all(sc);
    ex = (lane < tn) ? spec_expf(sc - m) : 0.0f;
    ls = wave_tree_sum64_all(ex);
}

// Attention item (query head h, chunk group g of ng) of one block: chunks
// c0 = 4g .. c0+ncg-1.  The four input waves split the group's scores (four
// positions per pass); then wave w accumulates V of chunk w/2 (and 2 + w/2)
// for dims 64*(w&1) + lane, each wave computing the softmax terms of its
// chunks itself (same operations on the same values, same bits).  A single
// group combines its chunks in LDS; with several groups every item publishes
// its chunks' partials (m, l, o) and the item of the last group combines all
// chunks of the head in ascending order as they arrive.  Same arithmetic as
// attention_kernel's STEP mode (hq_attention.hip).
__device__ void attention_item(const EngineParams& p, const hq_layer& Ly, int l, int h, int nc, int n, int pos,
                               const Slot& z, unsigned& budget)
{
    const int w = opaque_tid() / kWave;
    const int lane = lane_id();
    const int G = p.G;
    const int kvh = h / G;
    const int qd = p.heads * kD;
    const int ncg = nc;                      // every chunk of the context (nc <= kGroup)
    constexpr int c0 = 0;
    constexpr bool cur = true;               // the item holds the current position

    if (w == 0) {
        // q of head h (dims lane, lane+64); for the current group also k and
        // v of the kv head
        const float qn0 = gmem(Ly.q_norm)[lane], qn1 = gmem(Ly.q_norm)[lane + 64];
        const float kn0 = gmem(Ly.k_norm)[lane], kn1 = gmem(Ly.k_norm)[lane + 64];
        const float cs = gmem(p.rope_cos)[size_t(pos) * (kD / 2) + lane];
        const float sn = gmem(p.rope_sin)[size_t(pos) * (kD / 2) + lane];
        const __amdgpu_buffer_rsrc_t rq = buffer_rsrc(z.qkv());
        const uint32_t vo = uint32_t(lane) * 4u;
        const int sq_ = h * kD * 4;
        const int sk_ = (qd + kvh * kD) * 4;
        const int sv_ = (qd + (p.kv_heads + kvh) * kD) * 4;
        const uint32_t done = 1u;   // any non-zero word: nothing to wait for
        uint32_t eq0 = hs_load(rq, vo, sq_), eq1 = hs_load(rq, vo, sq_ + 256);
        uint32_t ek0 = done, ek1 = done, ev0 = done, ev1 = done;
        if (cur) {
            ek0 = hs_load(rq, vo, sk_);
            ek1 = hs_load(rq, vo, sk_ + 256);
            ev0 = hs_load(rq, vo, sv_);
            ev1 = hs_load(rq, vo, sv_ + 256);
        }
        unsigned spins = 0;
        while (budget != 0) {
            const int ready = int(hs_ready(eq0)) & int(hs_ready(eq1)) & int(hs_ready(ek0)) & int(hs_ready(ek1)) &
                              int(hs_ready(ev0)) & int(hs_ready(ev1));
            if (ready) break;
            __builtin_amdgcn_s_sleep(1);
            if (++spins == kSpinLimit) { budget = 0; atomicOr(p.status, HQ_STEP_SYNC); }
            compiler_fence();
            if (!hs_ready(eq0)) eq0 = hs_load(rq, vo, sq_);
            if (!hs_ready(eq1)) eq1 = hs_load(rq, vo, sq_ + 256);
            if (!hs_ready(ek0)) ek0 = hs_load(rq, vo, sk_);
            if (!hs_ready(ek1)) ek1 = hs_load(rq, vo, sk_ + 256);
            if (!hs_ready(ev0)) ev0 = hs_load(rq, vo, sv_);
            if (!hs_ready(ev1)) ev1 = hs_load(rq, vo, sv_ + 256);
        }
        if (w == 0) TRACE(l, 25);
        {
            // per-head RMSNorm + RoPE of q (as attention_kernel's STEP prologue)
            const float x0 = hs_value(eq0), x1 = hs_value(eq1);
            float s = __builtin_fmaf(x0, x0, 0.0f);
            s = __builtin_fmaf(x1, x1, s);
            const float ss = wave_tree_sum64_all(s);
            const float r = __builtin_sqrtf(ss / float(kD) + p.eps);
            const float y0 = (x0 / r) * qn0;
            const float y1 = (x1 / r) * qn1;
            S.aq[lane] = y0 * cs - y1 * sn;
            S.aq[lane + 64] = y1 * cs + y0 * sn;
        }
        if (cur) {
            // k (norm + RoPE) and v of this position, as fp16, into the row
            // of the last chunk; one query head of the group writes the cache
            const float x0 = hs_value(ek0), x1 = hs_value(ek1);
            float s = __builtin_fmaf(x0, x0, 0.0f);
            s = __builtin_fmaf(x1, x1, s);
            const float ss = wave_tree_sum64_all(s);
            const float r = __builtin_sqrtf(ss / float(kD) + p.eps);
            const float y0 = (x0 / r) * kn0;
            const float y1 = (x1 / r) * kn1;
            const uint16_t k0 = f32_to_f16(y0 * cs - y1 * sn), k1 = f32_to_f16(y1 * cs + y0 * sn);
            const uint16_t v0 = f32_to_f16(hs_value(ev0)), v1 = f32_to_f16(hs_value(ev1));
            KvBuf& lb = S.kv[ncg - 1];
            const int rr = pos - (nc - 1) * kAttnChunk;
            lb.k[rr * kD + lane] = k0;
            lb.k[rr * kD + lane + 64] = k1;
            lb.v[rr * kD + lane] = v0;
            lb.v[rr * kD + lane + 64] = v1;
            if (h % G == 0) {
                uint16_t* kl = p.keys + size_t(l) * size_t(p.kv_layer) + size_t(pos) * size_t(p.kv_stride) +
                               size_t(kvh) * kD;
                uint16_t* vl = p.values + size_t(l) * size_t(p.kv_layer) + size_t(pos) * size_t(p.kv_stride) +
                               size_t(kvh) * kD;
                kl[lane] = k0;
                kl[lane + 64] = k1;
                vl[lane] = v0;
                vl[lane + 64] = v1;
            }
        }
    }
    // the copy waves' K/V copies have landed (they issued them), q and the
    // current row are in place
    if (is_copy_wave(w)) wait_all_memory();
    __syncthreads();
    if (w == 0) TRACE(l, 26);

    // scores: pass P of a chunk covers its positions 4P .. 4P+3, 16 lanes
    // per position (8 dims each); wave w takes pass w of every chunk (the
    // rows of all chunks read first, then one independent chain per chunk)
    {
        const float scale = 1.0f / __builtin_sqrtf(float(kD));
        const int l16 = lane & 15;
        const int grp = lane >> 4;
        const int t = w * 4 + grp;
        float qv[8];
        const float4 qa = *reinterpret_cast<const float4*>(&S.aq[l16 * 8]);
        const float4 qb = *reinterpret_cast<const float4*>(&S.aq[l16 * 8 + 4]);
        qv[0] = qa.x; qv[1] = qa.y; qv[2] = qa.z; qv[3] = qa.w;
        qv[4] = qb.x; qv[5] = qb.y; qv[6] = qb.z; qv[7] = qb.w;
        // the code is specialized on the chunk count, so only the item's
        // chunks are computed (36 layers at context 64: 742 -> 737 us; the
        // GQA items' scores likewise: 905 -> 872 us at context 272)
        auto scores = [&](auto nc_const) {
            constexpr int NC = decltype(nc_const)::value;
            uint4 kw[NC];
            static_for<NC>([&](auto c) { kw[c] = *reinterpret_cast<const uint4*>(&S.kv[c].k[t * kD + l16 * 8]); });
            float pp[NC];
            static_for<NC>([&](auto c) {
                const uint32_t kk[4] = {kw[c].x, kw[c].y, kw[c].z, kw[c].w};
                float a = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    a = __builtin_fmaf(qv[2 * i], f16_to_f32(uint16_t(kk[i])), a);
                    a = __builtin_fmaf(qv[2 * i + 1], f16_to_f32(uint16_t(kk[i] >> 16)), a);
                }
                pp[c] = a;
            });
            static_for<NC>([&](auto c) { pp[c] = row_tree_sum16(pp[c]); });
            if (l16 == 0)
                static_for<NC>([&](auto c) {
                    const int tn = min(kAttnChunk, n - (c0 + c) * kAttnChunk);
                    S.as[c * kAttnChunk + t] = t < tn ? pp[c] * scale : -__builtin_inff();
                });
        };
        static_assert(kGroup == 4, "one specialization per chunk count");
        switch (ncg) {
        case 1: scores(std::integral_constant<int, 1>{}); break;
        case 2: scores(std::integral_constant<int, 2>{}); break;
        case 3: scores(std::integral_constant<int, 3>{}); break;
        default: scores(std::integral_constant<int, 4>{}); break;
        }
    }
    __syncthreads();
    if (w == 0) TRACE(l, 27);

    // chunk partials: wave w < 2*ncg takes dims 64*(w&1) + lane of chunk w/2
    // and computes the chunk's softmax terms itself (same operations on the
    // same values in both waves of a chunk, same bits)
    if (w < 2 * ncg) {
        const int ca = w >> 1;
        const int d = (w & 1) * kD / 2 + lane;
        float ma, ea, la;
        chunk_softmax(ca, min(kAttnChunk, n - (c0 + ca) * kAttnChunk), ma, ea, la);
        float oa = 0.0f, ob = 0.0f;
        v_chains<1>(&S.kv[ca].v[d], nullptr, ea, 0.0f, oa, ob);
        S.po[ca][d] = oa;
        if ((w & 1) == 0 && lane == 0) { S.pm[ca] = ma; S.pl[ca] = la; }
    }
    if (w == 0) TRACE(l, 28);
    __syncthreads();

    // combine (input waves, 32 dims per wave): the head's chunks are all
    // here: M = max m_c, then L and O over ascending chunks with
    // a_c = exp(m_c - M)
    if (w < kIWaves) {
        const int d = 32 * w + (lane & 31);
        float M = S.pm[0];
        for (int c = 1; c < ncg; ++c) M = fmaxf(M, S.pm[c]);
        float L = 0.0f, O = 0.0f;
        for (int c = 0; c < ncg; ++c) {
            const float al = spec_expf(S.pm[c] - M);
            L = __builtin_fmaf(al, S.pl[c], L);
            O = __builtin_fmaf(al, S.po[c][d], O);
        }
        if (lane < 32) hs_store(z.att() + size_t(h) * kD + d, O * (1.0f / L));
    }
    if (w == 0) TRACE(l, 29);
    // the item's LDS (K/V chunks, q, scores, partials) may be reused once
    // every wave is done
    __syncthreads();
}


// ---- GQA attention items (more than one chunk group per head) ---------------------
//
// At contexts of more than kGroup chunks the work item is (kv head, group of
// cg chunks) and serves the G query heads that share the kv head, so every
// K/V byte crosses one CU's memory pipe once (an item per query head would
// move it G times).  Each item publishes its chunks' partials (m, l, o) per
// query head as 64-bit {value, epoch} entries; afterwards every block
// combines the partials of its share of the attention output (gqa_combine),
// so no single block reads all of a head's partials.  Same arithmetic as the
// per-head items: the chunk terms, then the combine over ascending chunks.

// Chunks per GQA item: the fewest (up to kGroup) that give every item of the
// layer a block of its own.
__device__ __forceinline__ int gqa_group(int nc, int kv_heads, int nb)
{
    for (int cg = 1; cg < kGroup; ++cg)
        if (kv_heads * ((nc + cg - 1) / cg) <= nb) return cg;
    return kGroup;
}

// Softmax terms of the 64 scores at sc (lane t holds position t).
__device__ __forceinline__ void scores_softmax(const float* sc, int tn, float& m, float& ex, float& ls)
{
    const int lane = lane_id();
    const float v = sc[lane];
    m = wave_max64_all(v);
    ex = (lane < tn) ? spec_expf(v - m) : 0.0f;
    ls = wave_tree_sum64_all(ex);
}

__device__ void gqa_item(const EngineParams& p, const hq_layer& Ly, int l, int kvh, int g, int ngq, int cg, int nc,
                         int n, int pos, const Slot& z, uint32_t epoch_att, unsigned& budget)
{
    const int w = opaque_tid() / kWave;
    const int lane = lane_id();
    const int G = p.G;
    const int qd = p.heads * kD;
    const int c0 = g * cg;
    const int ncg = min(cg, nc - c0);
    const bool cur = g == ngq - 1;           // the group holding the current position
    constexpr int pstride = kD + 2;
    if (w == 0) TRACE(l, 48);

    if (w < G) {
        // wave w: query head kvh*G + w (dims lane, lane+64); wave 0 of the
        // current group also k and v of the kv head
        const int h = kvh * G + w;
        const bool kv = cur && w == 0;
        const float qn0 = gmem(Ly.q_norm)[lane], qn1 = gmem(Ly.q_norm)[lane + 64];
        const float kn0 = gmem(Ly.k_norm)[lane], kn1 = gmem(Ly.k_norm)[lane + 64];
        const float cs = gmem(p.rope_cos)[size_t(pos) * (kD / 2) + lane];
        const float sn = gmem(p.rope_sin)[size_t(pos) * (kD / 2) + lane];
        const __amdgpu_buffer_rsrc_t rq = buffer_rsrc(z.qkv());
        const uint32_t vo = uint32_t(lane) * 4u;
        const int sq_ = h * kD * 4;
        const int sk_ = (qd + kvh * kD) * 4;
        const int sv_ = (qd + (p.kv_heads + kvh) * kD) * 4;
        const uint32_t done = 1u;   // any non-zero word: nothing to wait for
        uint32_t eq0 = hs_load(rq, vo, sq_), eq1 = hs_load(rq, vo, sq_ + 256);
        uint32_t ek0 = done, ek1 = done, ev0 = done, ev1 = done;
        if (kv) {
            ek0 = hs_load(rq, vo, sk_);
            ek1 = hs_load(rq, vo, sk_ + 256);
            ev0 = hs_load(rq, vo, sv_);
            ev1 = hs_load(rq, vo, sv_ + 256);
        }
        unsigned spins = 0;
        while (budget != 0) {
            const int ready = int(hs_ready(eq0)) & int(hs_ready(eq1)) & int(hs_ready(ek0)) & int(hs_ready(ek1)) &
                              int(hs_ready(ev0)) & int(hs_ready(ev1));
            if (ready) break;
            __builtin_amdgcn_s_sleep(1);
            if (++spins == kSpinLimit) { budget = 0; atomicOr(p.status, HQ_STEP_SYNC); }
            compiler_fence();
            if (!hs_ready(eq0)) eq0 = hs_load(rq, vo, sq_);
            if (!hs_ready(eq1)) eq1 = hs_load(rq, vo, sq_ + 256);
            if (!hs_ready(ek0)) ek0 = hs_load(rq, vo, sk_);
            if (!hs_ready(ek1)) ek1 = hs_load(rq, vo, sk_ + 256);
            if (!hs_ready(ev0)) ev0 = hs_load(rq, vo, sv_);
            if (!hs_ready(ev1)) ev1 = hs_load(rq, vo, sv_ + 256);
        }
        {
            const float x0 = hs_value(eq0), x1 = hs_value(eq1);
            float s = __builtin_fmaf(x0, x0, 0.0f);
            s = __builtin_fmaf(x1, x1, s);
            const float ss = wave_tree_sum64_all(s);
            const float r = __builtin_sqrtf(ss / float(kD) + p.eps);
            const float y0 = (x0 / r) * qn0;
            const float y1 = (x1 / r) * qn1;
            S.gq[w][lane] = y0 * cs - y1 * sn;
            S.gq[w][lane + 64] = y1 * cs + y0 * sn;
        }
        if (kv) {
            const float x0 = hs_value(ek0), x1 = hs_value(ek1);
            float s = __builtin_fmaf(x0, x0, 0.0f);
            s = __builtin_fmaf(x1, x1, s);
            const float ss = wave_tree_sum64_all(s);
            const float r = __builtin_sqrtf(ss / float(kD) + p.eps);
            const float y0 = (x0 / r) * kn0;
            const float y1 = (x1 / r) * kn1;
            const uint16_t k0 = f32_to_f16(y0 * cs - y1 * sn), k1 = f32_to_f16(y1 * cs + y0 * sn);
            const uint16_t v0 = f32_to_f16(hs_value(ev0)), v1 = f32_to_f16(hs_value(ev1));
            KvBuf& lb = S.kv[ncg - 1];
            const int rr = pos - (nc - 1) * kAttnChunk;
            lb.k[rr * kD + lane] = k0;
            lb.k[rr * kD + lane + 64] = k1;
            lb.v[rr * kD + lane] = v0;
            lb.v[rr * kD + lane + 64] = v1;
            uint16_t* kl = p.keys + size_t(l) * size_t(p.kv_layer) + size_t(pos) * size_t(p.kv_stride) +
                           size_t(kvh) * kD;
            uint16_t* vl = p.values + size_t(l) * size_t(p.kv_layer) + size_t(pos) * size_t(p.kv_stride) +
                           size_t(kvh) * kD;
            kl[lane] = k0;
            kl[lane + 64] = k1;
            vl[lane] = v0;
            vl[lane + 64] = v1;
        }
    }
    if (w == 0) TRACE(l, 49);
    // the copy waves' K/V copies have landed (they issued them), the query
    // heads and the current row are in place
    if (is_copy_wave(w)) wait_all_memory();
    __syncthreads();
    if (w == 0) TRACE(l, 50);

    // scores: wave w takes positions 4w .. 4w+3 of every chunk (16 lanes per
    // position, 8 dims each) for every query head; the K rows are read once
    {
        const float scale = 1.0f / __builtin_sqrtf(float(kD));
        const int l16 = lane & 15;
        const int t = w * 4 + (lane >> 4);
        // specialized on the chunk count: only the item's chunks are computed
        auto scores = [&](auto nc_const) {
            constexpr int NC = decltype(nc_const)::value;
            uint4 kw[NC];
            static_for<NC>([&](auto c) { kw[c] = *reinterpret_cast<const uint4*>(&S.kv[c].k[t * kD + l16 * 8]); });
            for (int hh = 0; hh < G; ++hh) {
                float qv[8];
                const float4 qa = *reinterpret_cast<const float4*>(&S.gq[hh][l16 * 8]);
                const float4 qb = *reinterpret_cast<const float4*>(&S.gq[hh][l16 * 8 + 4]);
                qv[0] = qa.x; qv[1] = qa.y; qv[2] = qa.z; qv[3] = qa.w;
                qv[4] = qb.x; qv[5] = qb.y; qv[6] = qb.z; qv[7] = qb.w;
                float pp[NC];
                static_for<NC>([&](auto c) {
                    const uint32_t kk[4] = {kw[c].x, kw[c].y, kw[c].z, kw[c].w};
                    float a = 0.0f;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        a = __builtin_fmaf(qv[2 * i], f16_to_f32(uint16_t(kk[i])), a);
                        a = __builtin_fmaf(qv[2 * i + 1], f16_to_f32(uint16_t(kk[i] >> 16)), a);
                    }
                    pp[c] = row_tree_sum16(a);
                });
                if (l16 == 0)
                    static_for<NC>([&](auto c) {
                        const int tn = min(kAttnChunk, n - (c0 + c) * kAttnChunk);
                        S.gs[hh][c * kAttnChunk + t] = t < tn ? pp[c] * scale : -__builtin_inff();
                    });
            }
        };
        switch (ncg) {
        case 1: scores(std::integral_constant<int, 1>{}); break;
        case 2: scores(std::integral_constant<int, 2>{}); break;
        case 3: scores(std::integral_constant<int, 3>{}); break;
        default: scores(std::integral_constant<int, 4>{}); break;
        }
    }
    __syncthreads();
    if (w == 0) TRACE(l, 51);

    // chunk partials: task (head hh, chunk c, half of the dims); wave w takes
    // tasks w, w + 16, ...; each publishes its o values (and m, l) directly
    {
        const int ntask = 2 * G * ncg;
        for (int task = w; task < ntask; task += kWaves) {
            const int half = task & 1, hc = task >> 1, hh = hc / ncg, c = hc % ncg;
            const int tn = min(kAttnChunk, n - (c0 + c) * kAttnChunk);
            float m, ex, ls;
            scores_softmax(&S.gs[hh][c * kAttnChunk], tn, m, ex, ls);
            const int d = half * (kD / 2) + lane;
            float o = 0.0f, unused = 0.0f;
            v_chains<1>(&S.kv[c].v[d], nullptr, ex, 0.0f, o, unused);
            uint64_t* cp = p.ll_part + (size_t(kvh * G + hh) * size_t(p.max_chunks) + size_t(c0 + c)) * pstride;
            if (half == 0 && lane == 0) {
                ll_store(cp, m, epoch_att);
                ll_store(cp + 1, ls, epoch_att);
            }
            ll_store(cp + 2 + d, o, epoch_att);
        }
    }
    if (w == 0) TRACE(l, 52);
    // the item's LDS (K/V chunks, queries, scores) may be reused once every
    // wave is done
    __syncthreads();
    if (w == 0) TRACE(l, 53);
}

// Entries i < count (64-bit {value, epoch}, at src_of(i)) into dst[i] as
// floats, each polled until its epoch is current; input threads, NPT loads
// in flight per thread.
template <int NPT, class F>
__device__ __forceinline__ void gather_entries(int count, F&& src_of, float* dst, uint32_t epoch, unsigned& budget,
                                               int32_t* status)
{
    const int t = opaque_tid();
    for (int base = 0; base < count; base += NPT * kIThreads) {
        const uint64_t* a[NPT];
        uint64_t v[NPT];
        static_for<NPT>([&](auto j) {
            a[j] = src_of(min(base + t + j * kIThreads, count - 1));
            v[j] = __hip_atomic_load(const_cast<uint64_t*>(a[j]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        });
        unsigned spins = 0;
        while (budget != 0) {
            int pending = 0;
            static_for<NPT>([&](auto j) {
                pending |= int(base + t + j * kIThreads < count) & int(!ll_ready(v[j], epoch));
            });
            if (!pending) break;
            __builtin_amdgcn_s_sleep(1);
            if (++spins == kSpinLimit) { budget = 0; atomicOr(status, HQ_STEP_SYNC); }
            compiler_fence();
            static_for<NPT>([&](auto j) {
                if (base + t + j * kIThreads < count && !ll_ready(v[j], epoch))
                    v[j] = __hip_atomic_load(const_cast<uint64_t*>(a[j]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            });
        }
        static_for<NPT>([&](auto j) {
            const int i = base + t + j * kIThreads;
            if (i < count) dst[i] = bits_f32(uint32_t(v[j]));
        });
    }
}

// The attention output from the GQA items' chunk partials: block b owns
// output elements [e0, e0 + ne) of the qd = heads * D outputs (ne <= 256),
// input thread T element e0 + T (head h, dim d).  For its head: M = max of
// the chunks' m, a_c = exp(m_c - M), L = fmaf chain of a_c * l_c and O =
// fmaf chain of a_c * o_c[d] over ascending chunks, out = O * (1 / L).  The
// partials are staged in LDS (the K/V buffers, free after the items): in one
// gather when all chunks fit, else in batches after a first pass for M.
// The maxima are wave reductions and the a_c are computed by all threads;
// only the L and O chains run per element, as the spec orders them.  The
// four input waves meet at their barrier.
// The same combine for contexts of at most kSmallCombine chunks, with no
// barrier: input thread T (T < ne) polls the m and l entries of its head's
// chunks, forms M and every a_c itself (the same values in every thread of
// the head), runs the L chain, then polls its o entries and runs the O
// chain.  Same operations in the same order as gqa_combine (36 layers at
// context 272: 869 -> 840 us per launch, at 400: 873 -> 848 us).
constexpr int kSmallCombine = 8;
__device__ void gqa_combine_small(const EngineParams& p, int nc, const Slot& z, uint32_t epoch_att,
                                  unsigned& budget, int tl = -1)
{
    constexpr int pstride = kD + 2;
    const int t = opaque_tid();
    const int qd = p.heads * kD;
    const int e0 = split_begin(qd, blockIdx.x, gridDim.x);
    const int ne = split_begin(qd, blockIdx.x + 1, gridDim.x) - e0;
    if (t == 0) TRACE(tl, 54);
    if (t >= ne) return;
    const int e = e0 + t;
    const uint64_t* ph = p.ll_part + size_t(e / kD) * size_t(p.max_chunks) * pstride;
    auto poll = [&](uint64_t (&v)[kSmallCombine], int off) {
        static_for<kSmallCombine>([&](auto c) {
            v[c] = c < nc ? __hip_atomic_load(const_cast<uint64_t*>(ph + size_t(c) * pstride + off), __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT)
                          : 0;
        });
        unsigned spins = 0;
        while (budget != 0) {
            int pending = 0;
            static_for<kSmallCombine>([&](auto c) { pending |= int(c < nc) & int(!ll_ready(v[c], epoch_att)); });
            if (!pending) break;
            __builtin_amdgcn_s_sleep(1);
            if (++spins == kSpinLimit) { budget = 0; atomicOr(p.status, HQ_STEP_SYNC); }
            compiler_fence();
            static_for<kSmallCombine>([&](auto c) {
                if (c < nc && !ll_ready(v[c], epoch_att))
                    v[c] = __hip_atomic_load(const_cast<uint64_t*>(ph + size_t(c) * pstride + off), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
            });
        }
    };
    uint64_t vm[kSmallCombine], vl[kSmallCombine];
    poll(vm, 0);
    poll(vl, 1);
    if (t == 0) TRACE(tl, 55);
    float M = -__builtin_inff();
    static_for<kSmallCombine>([&](auto c) { if (c < nc) M = fmaxf(M, bits_f32(uint32_t(vm[c]))); });
    float a[kSmallCombine], L = 0.0f;
    static_for<kSmallCombine>([&](auto c) {
        if (c < nc) {
            a[c] = spec_expf(bits_f32(uint32_t(vm[c])) - M);
            L = __builtin_fmaf(a[c], bits_f32(uint32_t(vl[c])), L);
        }
    });
    uint64_t vo[kSmallCombine];
    poll(vo, 2 + e % kD);
    float O = 0.0f;
    static_for<kSmallCombine>([&](auto c) { if (c < nc) O = __builtin_fmaf(a[c], bits_f32(uint32_t(vo[c])), O); });
    if (t == 0) TRACE(tl, 56);
    hs_store(z.att() + e, O * (1.0f / L));
}

constexpr int kCombineChunks = 512;   // chunks per staged batch (at most)
__device__ void gqa_combine(const EngineParams& p, int nc, const Slot& z, uint32_t epoch_att, int& bseq,
                            unsigned& budget, int tl = -1)
{
    constexpr int pstride = kD + 2;
    constexpr int kStage = int(sizeof(S.kv) / (sizeof(float)));
    const int t = opaque_tid();
    const int w = t / kWave;
    const int qd = p.heads * kD;
    const int e0 = split_begin(qd, blockIdx.x, gridDim.x);
    const int ne = split_begin(qd, blockIdx.x + 1, gridDim.x) - e0;
    if (ne <= 0) return;   // (block-uniform: no input wave of the block takes the barriers below)
    const int h0 = e0 / kD;
    const int nh = (e0 + ne - 1) / kD - h0 + 1;        // 1 or 2 heads
    const int hi = (e0 + t) / kD - h0;                 // this thread's head (t < ne)
    float* stage = reinterpret_cast<float*>(&S.kv[0]);
    const uint64_t* part = p.ll_part;
    const size_t hstride = size_t(p.max_chunks) * pstride;
    const int cb2 = min(kCombineChunks, kStage / (2 * nh + ne));   // chunks per batch
    const bool single = nc <= cb2;
    // stage layout of a batch of nb chunks: m [nh][nb], l [nh][nb], o [ne][nb]
    auto gather_batch = [&](int cb, int nb, bool with_lo) {
        const int nm = nh * nb;
        const int count = with_lo ? (2 * nh + ne) * nb : nm;
        gather_entries<8>(count, [&](int i) {
            if (i < 2 * nm) {
                const int k = i / nb, c = cb + i % nb;       // k < nh: m of head k, else l of head k - nh
                return part + size_t(h0 + (k < nh ? k : k - nh)) * hstride + size_t(c) * pstride + size_t(k >= nh);
            }
            const int j = i - 2 * nm, el = j / nb, c = cb + j % nb;
            const int e = e0 + el;
            return part + size_t(e / kD) * hstride + size_t(c) * pstride + 2 + size_t(e % kD);
        }, stage, epoch_att, budget, p.status);
    };
    // M of each head (S.wmax[k]): wave k < nh reduces the m values of head k
    if (w == 0) TRACE(tl, 54);
    for (int cb = 0; cb < nc; cb += cb2) {
        const int nb = min(cb2, nc - cb);
        gather_batch(cb, nb, single);
        if (w == 0) TRACE(tl, 55);
        ibar(bseq, budget, p.status);
        if (w < nh) {
            float mm = -__builtin_inff();
            for (int c = lane_id(); c < nb; c += kWave) mm = fmaxf(mm, stage[w * nb + c]);
            mm = wave_max64_all(mm);
            if (lane_id() == 0) S.wmax[w] = fmaxf(cb == 0 ? -__builtin_inff() : S.wmax[w], mm);
        }
        ibar(bseq, budget, p.status);
    }
    float L = 0.0f, O = 0.0f;
    for (int cb = 0; cb < nc; cb += cb2) {
        const int nb = min(cb2, nc - cb);
        if (!single) {
            gather_batch(cb, nb, true);
            ibar(bseq, budget, p.status);
        }
        // a_c = exp(m_c - M) in place of the m values (every input thread)
        for (int i = t; i < nh * nb; i += kIThreads) stage[i] = spec_expf(stage[i] - S.wmax[i / nb]);
        ibar(bseq, budget, p.status);
        if (t < ne) {
            const float* sa = stage + hi * nb;
            const float* sl = stage + (nh + hi) * nb;
            const float* so = stage + 2 * nh * nb + t * nb;
            int c = 0;
            for (; c + 8 <= nb; c += 8) {
                float av[8], lv[8], ov[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) { av[j] = sa[c + j]; lv[j] = sl[c + j]; ov[j] = so[c + j]; }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    L = __builtin_fmaf(av[j], lv[j], L);
                    O = __builtin_fmaf(av[j], ov[j], O);
                }
            }
            for (; c < nb; ++c) {
                L = __builtin_fmaf(sa[c], sl[c], L);
                O = __builtin_fmaf(sa[c], so[c], O);
            }
        }
        ibar(bseq, budget, p.status);
    }
    if (w == 0) TRACE(tl, 56);
    if (t < ne) hs_store(z.att() + e0 + t, O * (1.0f / L));
}

// Per-head attention items (contexts of at most kGroup chunks): item h is
// query head h, so the G items that read the same K/V chunks are
// consecutive.  Round r of a layer gives block b item r*NB + k(b).  When
// G == 4 and NB is a multiple of 32 (blocks go to the 8 XCDs round robin,
// block b to XCD b % 8), k(b) places the four heads of one kv head on four
// blocks of one XCD: they run together and read their K/V through that
// XCD's L2 rather than four times over the fabric.  Otherwise k(b) = b.
__device__ __forceinline__ int item_slot(int b, int NB, int G)
{
    if (G != 4 || (NB & 31) != 0) return b;
    const int x = b & 7, rest = b >> 3;            // XCD, index within the XCD
    return (((rest >> 2) << 3) + x) * 4 + (rest & 3);
}

// All attention items of a layer for this block, run by all sixteen waves
// (the weight waves join after their qkv dots; every wave executes the same
// barriers).  The input waves copy each item's K/V chunks, the block's first
// item's copies having been started in P1.
__device__ void attention_phase(const EngineParams& p, const hq_layer& Ly, int l, int pos, const Slot& z,
                                uint32_t epoch_att, unsigned& budget)
{
    const int n = pos + 1;
    const int nc = (n + kAttnChunk - 1) / kAttnChunk;
    const int ng = (nc + kGroup - 1) / kGroup;
    if (ng > 1) {
        // GQA items, then every block combines its share of the output
        const int cg = gqa_group(nc, p.kv_heads, gridDim.x);
        const int ngq = (nc + cg - 1) / cg;
        const int gitems = p.kv_heads * ngq;
        for (int it = blockIdx.x; it < gitems; it += gridDim.x) {
            const int kvh = it / ngq, g = it % ngq;
            if (it != int(blockIdx.x) && is_copy_wave(opaque_tid() / kWave))
                prefetch_group(p, l, kvh, g * cg, min(cg, nc - g * cg), n, pos);
            gqa_item(p, Ly, l, kvh, g, ngq, cg, nc, n, pos, z, epoch_att, budget);
        }
        // (the input waves then combine the partials: gqa_combine, called
        // from the input role only, so the weight role's code holds none of it)
        return;
    }
    const int k = item_slot(blockIdx.x, gridDim.x, p.G);
    for (int h = k; h < p.heads; h += gridDim.x) {
        if (h != k && is_copy_wave(opaque_tid() / kWave)) prefetch_group(p, l, h / p.G, 0, nc, n, pos);
        attention_item(p, Ly, l, h, nc, n, pos, z, budget);
    }
}

// Publish the weight waves' results res[0, n) to dst (input threads t < n).
__device__ __forceinline__ void publish_rows(uint32_t* dst, int n)
{
    const int t = opaque_tid();
    for (int i = t; i < n; i += kIThreads) hs_store(dst + i, S.res[i]);
}

__device__ __forceinline__ void input_role(const EngineParams& p, const Rows& R, int pos, uint32_t base, int set,
                                           unsigned& budget)
{
    const int t0 = threadIdx.x;
    const int H = p.H;
    const int qd = p.heads * kD;
    const int nown = R.h1 - R.h0;
    int bseq = 0;   // input-barrier count
    // layer 0's input: x, or the embedding row of the current token
    // (element i: nibble i of the row, low nibble first, times its scale,
    // as the embedding kernel computes it; an out-of-range token flags the
    // status and reads row 0)
    int tok = 0;
    if (p.token != nullptr) {
        tok = *p.token;
        if (tok < 0 || tok >= p.vocab) {
            if (blockIdx.x == 0 && t0 == 0) atomicOr(p.status, HQ_STEP_BAD_TOKEN);
            tok = 0;
        }
    }
    auto layer_input = [&](int i) -> float {
        if (p.token == nullptr) return p.x[i];
        const uint8_t b = p.emb[size_t(tok) * size_t(H >> 1) + size_t(i >> 1)];
        const int v = (i & 1) ? int(int8_t(b)) >> 4 : int(int8_t(uint8_t(b << 4))) >> 4;
        return float(v) * p.emb_scales[tok];
    };
    float xown = t0 < nown ? layer_input(R.h0 + t0) : 0.0f;

#pragma unroll 1
    for (int l = 0; l < p.L; ++l) {
        const int t = opaque_tid();   // (addresses from it are not hoisted out of the loop)
        const hq_layer& Ly = S.lay[l];
        const uint32_t E = base + 5u * uint32_t(l);
        const Slot z = slot_of(p, set, l);
        const uint32_t* x5_prev = slot_of(p, set, l > 0 ? l - 1 : 0).x5();

        // ---- P1: RMSNorm(input) -> quant -> (qkv) -------------------------------------
        TRACE(l, 0);
        {
            float gin[kHidNPT];
            load_gamma(Ly.input_norm, H, gin);
            float xin[kHidNPT];
            if (l == 0) {
#pragma unroll
                for (int j = 0; j < kHidNPT; ++j) xin[j] = t + kIThreads * j < H ? layer_input(t + kIThreads * j) : 0.0f;
            } else {
                watch_last(x5_prev, H, budget, p.status);
                TRACE(l, 1);
                poll_into<kHidNPT>(x5_prev, H, xin, budget, p.status);
            }
            post_hs();
            TRACE(l, 2);
            const float act = rmsnorm_quant(xin, H, gin, p.eps, kQkvLPR * kQkvC * 32, bseq, budget, p.status, l, 37);
            post_xq(act);
            TRACE(l, 3);
        }
        block_sync();   // the weight waves' results in S.res
        TRACE(l, 4);
        publish_rows(z.qkv() + R.q0, R.q1 - R.q0);

        // ---- P2: attention ------------------------------------------------------------
        attention_phase(p, Ly, l, pos, z, E + 2, budget);
        {
            const int nc = (pos + 1 + kAttnChunk - 1) / kAttnChunk;
            if (nc > kSmallCombine) gqa_combine(p, nc, z, E + 2, bseq, budget, l);
            else if (nc > kGroup) gqa_combine_small(p, nc, z, E + 2, budget, l);
        }

        // ---- P3: quant -> (o) -> residual ---------------------------------------------
        float gpost[kHidNPT];
        {
            TRACE(l, 5);
            if (nown > 0) {
                float att[kAttNPT];
                watch_last(z.att(), qd, budget, p.status);
                TRACE(l, 6);
                poll_into<kAttNPT>(z.att(), qd, att, budget, p.status);
                post_hs();
                load_gamma(Ly.post_norm, H, gpost);
                const float act = quantize(att, qd, kOLPR * kOC * 32, bseq, budget, p.status);
                post_xq(act);
            } else {
                // (block-uniform) no o rows here: the weight waves' o dot
                // runs on the previous input and stores nothing, so only
                // the counters move on
                post_hs();
                load_gamma(Ly.post_norm, H, gpost);
                post_xq(0.0f);
            }
            TRACE(l, 7);
        }
        block_sync();   // the weight waves' results in S.res
        TRACE(l, 8);
        if (t < nown) {
            xown = xown + S.res[t];
            hs_store(z.x3() + R.h0 + t, xown);
        }

        // ---- P4: RMSNorm(post) -> quant -> (gate_up, SwiGLU) --------------------------
        {
            float xp[kHidNPT];
            watch_last(z.x3(), H, budget, p.status);
            TRACE(l, 9);
            poll_into<kHidNPT>(z.x3(), H, xp, budget, p.status);
            post_hs();
            const float act = rmsnorm_quant(xp, H, gpost, p.eps, kGuLPR * kGuC * 32, bseq, budget, p.status, l, 32);
            post_xq(act);
            TRACE(l, 10);
        }
        block_sync();   // the weight waves' results in S.res
        TRACE(l, 11);
        // The SwiGLU output is handed on as fp32 values: every block reads
        // the whole vector, takes its maximum |value| (order-free) and
        // quantizes it into its own S.xq, so one hand-off carries both the
        // act scale and the down GEMV's input.
        const int na = R.g1 - R.g0;
        if (t < na) hs_store(z.act() + R.g0 + t, S.res[t]);

        // ---- P5: quant (all waves) -> (down) -> residual --------------------------------
        act_phase(p, l, z.act(), budget);
        post_hs();
        TRACE(l, 13);
        block_sync();   // the weight waves' results in S.res
        TRACE(l, 14);
        if (t < nown) {
            xown = xown + S.res[t];
            if (l + 1 < p.L) hs_store(z.x5() + R.h0 + t, xown);
            else p.x[R.h0 + t] = xown;
        }
    }
}

}  // namespace

__global__ __launch_bounds__(eng::kThreads) void engine_kernel(EngineParams p)
{
    const int tid = threadIdx.x;
    const int b = blockIdx.x;
    const int NB = gridDim.x;

    const int pos = *p.position;
    if (pos < 0 || pos >= p.capacity) {
        if (b == 0 && tid == 0) atomicOr(p.status, HQ_STEP_FULL);
        return;
    }
    const uint32_t base = *p.epoch;
    // the hand-off set of this launch (launches alternate between two)
    const int set = int((base / (5u * uint32_t(p.L))) & 1u);
    Rows R;
    R.q0 = split_begin(p.qkv_rows, b, NB);
    R.q1 = split_begin(p.qkv_rows, b + 1, NB);
    // The hidden rows (o, down and the residual entries) and the SwiGLU rows
    // go to the blocks without attention items when those can hold them
    // (one hidden row and four SwiGLU pairs per weight wave): an item block
    // is the last to post its o and gate_up inputs (36 layers at context
    // 64: its residual entries arrived about 1.5 us after the others' in
    // every layer).  A block without rows gets empty ranges at H - 1 and I:
    // its loads clamp to valid rows and it stores nothing.  SwiGLU rows go
    // in whole groups of 8, so a block's quantized outputs fill whole 8-byte
    // groups of the de-interleaved activation layout.
    const int nit = item_block_prefix(p, pos);
    const int nfree = NB - nit;
    const int ng8 = p.I / 8;
    if (nit > 0 && nfree > 0 && (p.H + nfree - 1) / nfree <= min(kWWaves, kMaxOwn) &&
        8 * ((ng8 + nfree - 1) / nfree) <= min(kWWaves * 4, kMaxRes)) {
        const bool item = b < nit;
        const int j = b - nit;
        R.h0 = item ? p.H - 1 : split_begin(p.H, j, nfree);
        R.h1 = item ? p.H - 1 : split_begin(p.H, j + 1, nfree);
        R.g0 = item ? p.I : 8 * split_begin(ng8, j, nfree);
        R.g1 = item ? p.I : 8 * split_begin(ng8, j + 1, nfree);
    } else {
        R.h0 = split_begin(p.H, b, NB);
        R.h1 = split_begin(p.H, b + 1, NB);
        R.g0 = 8 * split_begin(ng8, b, NB);
        R.g1 = 8 * split_begin(ng8, b + 1, NB);
    }
    {
        constexpr int kWords = sizeof(hq_layer) / sizeof(uint64_t);
        const uint64_t* src = reinterpret_cast<const uint64_t*>(p.layers);
        uint64_t* dst = reinterpret_cast<uint64_t*>(S.lay);
        for (int i = tid; i < p.L * kWords; i += kThreads) dst[i] = src[i];
    }
    {
        // This block's share of the other set (written by the previous
        // launch, which has finished) back to empty, before any weight load
        // is issued; the next launch uses that set.
        const size_t words = size_t(p.L) * size_t(p.hs_layer);
        uint32_t* o = p.hs + size_t(set ^ 1) * words;
        const size_t c0 = words * size_t(b) / size_t(NB), c1 = words * size_t(b + 1) / size_t(NB);
        for (size_t i = c0 + size_t(tid); i < c1; i += kThreads)
            __hip_atomic_store(o + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (tid == 0) {
        S.xq_seq = 0;
        S.ibar = 0;
        S.hs = 0;
    }
    __syncthreads();
    unsigned budget = 1;   // nonzero while this thread still waits (see kSpinLimit)
    const int wave = tid / kWave;
#ifdef HQ_ENGINE_TRACE
    for (int i = tid; i < kTraceWords; i += kThreads) S.trace[i] = 0;
    __syncthreads();
#endif
    if (wave >= kIWaves) weight_role(p, R, wave - kIWaves, pos, base, set, budget);
    else input_role(p, R, pos, base, set, budget);
#ifdef HQ_ENGINE_TRACE
    __syncthreads();
    for (int i = tid; i < kTraceWords; i += kThreads) p.trace[size_t(b) * kTraceWords + i] = S.trace[i];
#endif
    // (the thread index re-read here: holding it across the layer loop costs a register)
    if (blockIdx.x == 0 && opaque_tid() == 0) *p.epoch = base + 5u * uint32_t(p.L);
}

// ---- host ---------------------------------------------------------------------

bool engine_fits(const hq_model* m)
{
    using namespace eng;
    if (m->head_dim != kD) return false;
    const int G = m->heads / m->kv_heads;
    if (G > kG || G > kIWaves || m->heads % m->kv_heads) return false;
    if (m->layers > kMaxLayers) return false;
    const int H = m->hidden, I = m->intermediate, qd = m->heads * kD;
    if (H > kMaxHidden || I > kMaxVec || qd > kMaxVec) return false;
    if (H > kIThreads * kHidNPT || qd > kIThreads * kAttNPT || I > kThreads * kActNPT) return false;
    if (I % 8) return false;   // SwiGLU rows are handed on in groups of 8
    if ((H >> 5) > kQkvLPR * kQkvC || (H >> 5) > kGuLPR * kGuC) return false;
    if ((qd >> 5) > kOLPR * kOC || (I >> 5) > kDownLPR * kDownC) return false;
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
    int nb = min(min(cus[dev], m->hidden), min(qrows, m->intermediate / 8));
    // per-block capacities of the weight waves and the residual rows
    auto ceil_div = [](int a, int b) { return (a + b - 1) / b; };
    if (ceil_div(qrows, nb) > kWWaves * (kWave / kQkvLPR) || ceil_div(m->hidden, nb) > kWWaves ||
        ceil_div(m->hidden, nb) > kMaxOwn || 8 * ceil_div(m->intermediate / 8, nb) > kWWaves * 4 ||
        ceil_div(qrows, nb) > kMaxRes || 8 * ceil_div(m->intermediate / 8, nb) > kMaxRes ||
        ceil_div(m->heads * kD, nb) > kIThreads)   // the attention combine's elements per block
        return 0;
    return nb;
}

size_t engine_trace_bytes(const hq_model* m)
{
    (void)m;
#ifdef HQ_ENGINE_TRACE
    return size_t(1024) * eng::kTraceWords * sizeof(uint32_t);
#else
    return 0;
#endif
}

static int engine_layer_words(const hq_model* m)
{
    const int qd = m->heads * m->head_dim;
    const int qrows = qd + 2 * m->kv_heads * m->head_dim;
    return 2 * m->hidden + qrows + qd + m->intermediate;
}

size_t engine_handoff_bytes(const hq_model* m)
{
    return size_t(2) * size_t(m->layers) * size_t(engine_layer_words(m)) * 4;
}

hipError_t launch_engine(const hq_model* m, const hq_state* st, uint32_t* hs, uint32_t* epoch,
                         uint64_t* part, int max_chunks, int nb, uint32_t* trace, bool embed, hipStream_t s)
{
    EngineParams p{};
    if (embed) {
        p.token = st->token;
        p.emb = m->embedding;
        p.emb_scales = m->embedding_scales;
        p.vocab = m->vocab;
    }
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
    p.hs = hs;
    p.hs_layer = engine_layer_words(m);
    p.epoch = epoch;
    p.ll_part = part;
    p.max_chunks = max_chunks;
    p.trace = trace;
    hipLaunchKernelGGL(engine_kernel, dim3(nb), dim3(eng::kThreads), 0, s, p);
    return hipGetLastError();
}

}  // namespace hq
