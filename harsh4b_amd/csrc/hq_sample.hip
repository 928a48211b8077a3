// hq_sample.hip - the stochastic sampler of the reference's CPU runner
// (sample_logits, cpu_lightspark.py:706-726 in the reference repository) on
// gfx950: repetition penalty, temperature, top-k, softmax, top-p and the
// inverse-cdf draw of numpy's Generator.choice, given the uniform draw u.
//
//   1. block b loads logits[b*S, (b+1)*S) into LDS and applies the penalty
//      there: v[id] = logits[id] > 0 ? logits[id] / rp : logits[id] * rp for
//      every id of `generated` in its slice (a repeated id writes the same
//      value again)
//   2. it turns v_i / temperature into 64-bit sort keys (value descending,
//      NaN last, index ascending; the value is recoverable from the key)
//      and radix-selects its k smallest keys, 8 bits per pass, into a
//      candidate list in global memory
//   3. the last block to finish (a ticket counter) selects the k smallest of
//      all candidates the same way, sorts those k, and runs softmax / top-p
//      / cdf in the reference's order with the repo's exp and numpy's float32
//      summation order; the ordered sums run on thread 0
// The result equals the oracle's or_sample_token bit for bit (ids,
// probabilities, token).  One launch per token.
#include "hq_device.h"
#include "hq_internal.h"

namespace hq {

constexpr int kSampleThreads = 1024;
constexpr int kSampleSlice = 4096;               // logits per block; keys the LDS array holds
constexpr int kSampleMaxK = kSampleSlice / 2;    // the last block's chunks add at least k keys

// Sort key: ascending key order = value descending (NaN last), then index
// ascending.  -0 ranks (and is recovered) as +0.
__device__ __forceinline__ uint64_t sample_key(float v, int i)
{
    uint32_t hi;
    if (v != v) {
        hi = 0xFFFFFFFFu;
    } else {
        uint32_t u = f32_bits(v);
        if (u == 0x80000000u) u = 0;
        const uint32_t asc = (u & 0x80000000u) ? ~u : (u | 0x80000000u);   // ascending with the value
        hi = ~asc;
    }
    return (uint64_t(hi) << 32) | uint32_t(i);
}

// Past the end of the logits: after every real key (NaN keys included,
// whose indices are < n) and distinct, as the radix select needs.
__device__ __forceinline__ uint64_t pad_key(int i) { return (uint64_t(0xFFFFFFFFu) << 32) | uint32_t(i); }

__device__ __forceinline__ float key_value(uint64_t key)
{
    const uint32_t asc = ~uint32_t(key >> 32);
    return __uint_as_float((asc & 0x80000000u) ? (asc & 0x7FFFFFFFu) : ~asc);
}

__device__ __forceinline__ int key_index(uint64_t key) { return int(uint32_t(key)); }

__device__ __forceinline__ void publish_u64(uint64_t* p, uint64_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t read_u64(const uint64_t* p)
{
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct SampleShared {
    uint64_t key[kSampleSlice];
    union {
        float v[kSampleSlice];                          // the slice's values (phase 1)
        struct {
            uint64_t win[kSampleMaxK];                  // selected keys (last block)
            float p[kSampleMaxK];
            float drop[kSampleMaxK];
        } f;
    } u;
    int hist[256];
    int digit, before, done, count, ticket;
    float total;
};

// The k smallest of the `count` keys S.key[0..count) (k <= count; the keys
// must be distinct, or the last bin could hand out more than k),
// written unordered to out[0..k) by LDS-atomic positions.  Radix select on
// 8-bit digits from the top: each pass histograms the keys that share the
// digits chosen so far and picks the digit bin holding the k-th key; when
// that bin is taken whole the selection stops early.  Every thread of the
// block calls it; out may be global memory (published with agent scope).
template <bool GLOBAL>
__device__ void select_k(SampleShared& S, int count, int k, uint64_t* out)
{
    const int t = threadIdx.x;
    uint64_t prefix = 0, mask = 0;
    int need = k;
    for (int shift = 56; shift >= 0; shift -= 8) {
        if (t < 256) S.hist[t] = 0;
        __syncthreads();
        for (int j = t; j < count; j += kSampleThreads) {
            const uint64_t x = S.key[j];
            if ((x & mask) == prefix) atomicAdd(&S.hist[int(x >> shift) & 255], 1);
        }
        __syncthreads();
        if (t < 64) {
            int c[4], sum = 0;
            for (int j = 0; j < 4; ++j) {
                c[j] = S.hist[4 * t + j];
                sum += c[j];
            }
            int incl = sum;
            for (int o = 1; o < 64; o <<= 1) {
                const int y = __shfl_up(incl, o, 64);
                if (t >= o) incl += y;
            }
            int before = incl - sum;
            if (before < need && need <= incl) {
                for (int j = 0; j < 4; ++j) {
                    if (need <= before + c[j]) {
                        S.digit = 4 * t + j;
                        S.before = before;
                        S.done = (need - before) == c[j];
                        break;
                    }
                    before += c[j];
                }
            }
        }
        __syncthreads();
        need -= S.before;
        prefix |= uint64_t(S.digit) << shift;
        mask |= uint64_t(255) << shift;
        const bool done = S.done;
        __syncthreads();                       // digit/before/done are rewritten next pass
        if (done) break;
    }
    if (t == 0) S.count = 0;
    __syncthreads();
    for (int j = t; j < count; j += kSampleThreads) {
        const uint64_t x = S.key[j];
        if ((x & mask) <= prefix) {
            const int pos = atomicAdd(&S.count, 1);
            if (GLOBAL) publish_u64(out + pos, x);
            else out[pos] = x;
        }
    }
    __syncthreads();
}

// Ascending bitonic sort of S.key[0..n) (n a power of two <= kSampleSlice).
__device__ void bitonic_sort(uint64_t* key, int n)
{
    for (int k = 2; k <= n; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < n; i += kSampleThreads) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const uint64_t a = key[i], b = key[ixj];
                    if ((a > b) == ((i & k) == 0)) {
                        key[i] = b;
                        key[ixj] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
}

// numpy's float32 add.reduce order (pairwise_sum of umath's loops_utils):
// < 8 values in order, <= 128 in eight running sums, larger halves split at
// a multiple of 8 below n/2 and summed left + right.  The recursion runs on
// an explicit stack; n <= kSampleMaxK needs at most 6 frames.
__device__ float pairwise_leaf(const float* a, int n)
{
    if (n < 8) {
        float r = 0.0f;
        for (int i = 0; i < n; ++i) r += a[i];
        return r;
    }
    float r[8];
    for (int j = 0; j < 8; ++j) r[j] = a[j];
    int i = 8;
    for (; i < n - (n % 8); i += 8)
        for (int j = 0; j < 8; ++j) r[j] += a[i + j];
    float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < n; ++i) res += a[i];
    return res;
}

__device__ float pairwise_sum_f32(const float* a, int n)
{
    constexpr int kDepth = 8;
    int off[kDepth], len[kDepth], state[kDepth];
    float left[kDepth];
    int sp = 0;
    off[0] = 0;
    len[0] = n;
    state[0] = 0;
    float ret = 0.0f;
    while (sp >= 0) {
        if (len[sp] <= 128) {
            ret = pairwise_leaf(a + off[sp], len[sp]);
            --sp;
            continue;
        }
        int n2 = len[sp] / 2;
        n2 -= n2 % 8;
        if (state[sp] == 0) {                 // left half
            state[sp] = 1;
            off[sp + 1] = off[sp];
            len[sp + 1] = n2;
            state[sp + 1] = 0;
            ++sp;
        } else if (state[sp] == 1) {          // right half
            left[sp] = ret;
            state[sp] = 2;
            off[sp + 1] = off[sp] + n2;
            len[sp + 1] = len[sp] - n2;
            state[sp + 1] = 0;
            ++sp;
        } else {
            ret = left[sp] + ret;
            --sp;
        }
    }
    return ret;
}

struct SampleParams {
    const float* logits;
    const int32_t* generated;
    const double* u;
    int32_t* out_token;
    int32_t* ids_out;
    float* probs_out;
    uint64_t* cand;       // gridDim.x * k candidate keys
    int* counter;         // zero between calls (the last block resets it)
    int n, n_generated, k;
    float rp, temperature, top_p;
};

// softmax / top-p / Generator.choice over the k sorted keys S.key[0..k).
__device__ void sample_finish(SampleShared& S, const SampleParams& p)
{
    const int t = threadIdx.x;
    const int k = p.k;
    float* prob = S.u.f.p;
    float* drop = S.u.f.drop;
    const float top = key_value(S.key[0]);
    for (int i = t; i < k; i += kSampleThreads) prob[i] = spec_expf(key_value(S.key[i]) - top);
    __syncthreads();
    if (t == 0) S.total = pairwise_sum_f32(prob, k);
    __syncthreads();
    for (int i = t; i < k; i += kSampleThreads) prob[i] = prob[i] / S.total;
    __syncthreads();
    if (p.top_p < 1.0f) {
        if (t == 0) {
            float c = 0.0f;
            for (int i = 0; i < k; ++i) {
                c = c + prob[i];
                drop[i] = c - prob[i];
            }
        }
        __syncthreads();
        for (int i = t; i < k; i += kSampleThreads)
            if (drop[i] >= p.top_p) prob[i] = 0.0f;
        __syncthreads();
        if (t == 0) S.total = pairwise_sum_f32(prob, k);
        __syncthreads();
        for (int i = t; i < k; i += kSampleThreads) prob[i] = prob[i] / S.total;
        __syncthreads();
    }
    if (t == 0) {
        // Generator.choice: cdf = cumsum(double(p)) / its last entry; the
        // token is ids[#{i : cdf_i <= u}]
        double last = 0.0;
        for (int i = 0; i < k; ++i) last = last + double(prob[i]);
        const double draw = *p.u;
        double cdf = 0.0;
        int index = 0;
        for (int i = 0; i < k; ++i) {
            cdf = cdf + double(prob[i]);
            if (cdf / last <= draw) index = i + 1;
        }
        if (index >= k) index = k - 1;
        *p.out_token = key_index(S.key[index]);
    }
    if (p.ids_out)
        for (int i = t; i < k; i += kSampleThreads) p.ids_out[i] = key_index(S.key[i]);
    if (p.probs_out)
        for (int i = t; i < k; i += kSampleThreads) p.probs_out[i] = prob[i];
}

__global__ __launch_bounds__(kSampleThreads) void sample_kernel(SampleParams p)
{
    __shared__ SampleShared S;
    const int t = threadIdx.x;
    const int k = p.k;
    const int base = blockIdx.x * kSampleSlice;
    // 1. the slice's values, penalised
    for (int j = t; j < kSampleSlice; j += kSampleThreads) {
        const int i = base + j;
        S.u.v[j] = i < p.n ? p.logits[i] : 0.0f;
    }
    __syncthreads();
    if (p.rp != 1.0f) {
        for (int g = t; g < p.n_generated; g += kSampleThreads) {
            const int id = p.generated[g];
            if (id < base || id >= base + kSampleSlice || id >= p.n) continue;
            const float x = p.logits[id];
            S.u.v[id - base] = x > 0.0f ? x / p.rp : x * p.rp;
        }
        __syncthreads();
    }
    // 2. keys, and this slice's k smallest into the candidate list
    for (int j = t; j < kSampleSlice; j += kSampleThreads) {
        const int i = base + j;
        S.key[j] = i < p.n ? sample_key(S.u.v[j] / p.temperature, i) : pad_key(i);
    }
    __syncthreads();
    select_k<true>(S, kSampleSlice, k, p.cand + size_t(blockIdx.x) * k);
    // 3. the last block to finish reduces every slice's candidates
    wait_all_memory();                         // this thread's candidate stores have completed
    __syncthreads();
    if (t == 0) S.ticket = atomicAdd(p.counter, 1);
    __syncthreads();
    if (S.ticket != int(gridDim.x) - 1) return;
    const int total = int(gridDim.x) * k;
    int have = 0;
    for (int off = 0; off < total;) {
        const int chunk = min(total - off, kSampleSlice - have);
        for (int j = t; j < chunk; j += kSampleThreads) S.key[have + j] = read_u64(p.cand + off + j);
        off += chunk;
        const int count = have + chunk;
        __syncthreads();
        if (count > k) {
            select_k<false>(S, count, k, S.u.f.win);
            for (int j = t; j < k; j += kSampleThreads) S.key[j] = S.u.f.win[j];
            __syncthreads();
            have = k;
        } else {
            have = count;
        }
    }
    int m = 1;
    while (m < k) m <<= 1;
    for (int j = k + t; j < m; j += kSampleThreads) S.key[j] = ~uint64_t(0);
    __syncthreads();
    bitonic_sort(S.key, m);
    sample_finish(S, p);
    if (t == 0) publish_i(p.counter, 0);
}

static size_t al256s(size_t v) { return (v + 255) & ~size_t(255); }

static int sample_slices(int n) { return (n + kSampleSlice - 1) / kSampleSlice; }

}  // namespace hq

using namespace hq;

extern "C" size_t hq_sample_workspace_bytes(int n, int top_k)
{
    if (n <= 0 || top_k <= 0) return 0;
    const int k = top_k < n ? top_k : n;
    return 256 + al256s(size_t(sample_slices(n)) * size_t(k) * 8);   // counter, then candidates
}

extern "C" int hq_sample_token(const float* logits, int n, const int32_t* generated, int n_generated,
                               float repetition_penalty, float temperature, int top_k, float top_p,
                               const double* u, int32_t* out_token, int32_t* ids_out, float* probs_out,
                               void* workspace, void* stream)
{
    if (!logits || !u || !out_token || !workspace || n <= 0 || n_generated < 0) return HQ_ERR_ARG;
    if (n_generated > 0 && !generated) return HQ_ERR_ARG;
    if (top_k < 1 || top_k > kSampleMaxK) return HQ_ERR_ARG;
    if (!(temperature > 0.0f) || !(repetition_penalty > 0.0f) || !(top_p > 0.0f)) return HQ_ERR_ARG;
    if (reinterpret_cast<uintptr_t>(workspace) & 255u) return HQ_ERR_ALIGN;
    SampleParams p;
    p.logits = logits;
    p.generated = generated;
    p.u = u;
    p.out_token = out_token;
    p.ids_out = ids_out;
    p.probs_out = probs_out;
    p.n = n;
    p.n_generated = n_generated;
    p.k = top_k < n ? top_k : n;
    p.rp = repetition_penalty;
    p.temperature = temperature;
    p.top_p = top_p;
    const int blocks = sample_slices(n);
    char* ws = static_cast<char*>(workspace);
    p.counter = reinterpret_cast<int*>(ws);     // at a fixed place: calls with any n and k share it
    p.cand = reinterpret_cast<uint64_t*>(ws + 256);
    hipLaunchKernelGGL(sample_kernel, dim3(blocks), dim3(kSampleThreads), 0, static_cast<hipStream_t>(stream), p);
    return hipGetLastError() == hipSuccess ? HQ_OK : HQ_ERR_LAUNCH;
}
