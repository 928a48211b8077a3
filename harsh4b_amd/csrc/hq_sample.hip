// hq_sample.hip - the stochastic sampler of the reference's CPU runner
// (sample_logits, cpu_lightspark.py:706-726 in the reference repository) on
// gfx950: repetition penalty, temperature, top-k, softmax, top-p and the
// inverse-cdf draw of numpy's Generator.choice, given the uniform draw u.
//
//   1. values = logits                                   (sample_copy_kernel)
//   2. values[id] = logits[id] > 0 ? logits[id] / rp : logits[id] * rp for
//      every id of `generated` (a repeated id writes the same value again)
//   3. v_i = values[i] / temperature; each block sorts its slice of v by
//      (value descending, NaN last, index ascending) in LDS and keeps its
//      first k entries as a sorted list                  (sample_block_kernel)
//   4. while more than one list is left, each block sorts the union of
//      kSampleSlice / k lists and keeps its first k      (sample_merge_kernel)
//   5. one block runs softmax / top-p / cdf on the k survivors in the
//      reference's order, with the repo's exp and numpy's float32 summation
//      order; the ordered sums run on thread 0           (sample_finish_kernel)
// The result equals the oracle's or_sample_token bit for bit (ids,
// probabilities, token).
#include "hq_device.h"
#include "hq_internal.h"

namespace hq {

constexpr int kSampleBlock = 1024;      // threads of the slice and merge sorts
constexpr int kSampleSlice = 4096;      // keys one sort holds (32 KiB of LDS)
constexpr int kSampleFinish = 1024;     // threads of the finish kernel
constexpr int kSampleMaxK = kSampleSlice / 2;   // a merge joins at least two lists

// Sort key: ascending key order = value descending (NaN last), then index
// ascending.  -0 and +0 rank as equal values.  ~0 pads a slice: it sorts
// after every real key.
__device__ __forceinline__ uint64_t sample_key(float v, int i)
{
    uint32_t u = f32_bits(v);
    uint32_t hi;
    if (v != v) {
        hi = 0xFFFFFFFFu;
    } else {
        if (u == 0x80000000u) u = 0;
        const uint32_t asc = (u & 0x80000000u) ? ~u : (u | 0x80000000u);   // ascending with the value
        hi = ~asc;                                                             // descending
    }
    return (uint64_t(hi) << 32) | uint32_t(i);
}

// Ascending bitonic sort of kSampleSlice keys in LDS by kSampleBlock threads.
__device__ void bitonic_sort(uint64_t* key)
{
    for (int k = 2; k <= kSampleSlice; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < kSampleSlice; i += kSampleBlock) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const uint64_t a = key[i], b = key[ixj];
                    const bool up = (i & k) == 0;
                    if ((a > b) == up) {
                        key[i] = b;
                        key[ixj] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
}

__global__ __launch_bounds__(kBlock) void sample_copy_kernel(const float* logits, int n, float* values)
{
    for (int i = blockIdx.x * kBlock + threadIdx.x; i < n; i += gridDim.x * kBlock) values[i] = logits[i];
}

// A repeated id writes the same value again, so duplicates need no removal.
__global__ __launch_bounds__(kBlock) void sample_penalty_kernel(const float* logits, int n, const int32_t* generated,
                                                                int n_generated, float rp, float* values)
{
    for (int g = blockIdx.x * kBlock + threadIdx.x; g < n_generated; g += gridDim.x * kBlock) {
        const int id = generated[g];
        if (id < 0 || id >= n) continue;
        const float x = logits[id];
        values[id] = x > 0.0f ? x / rp : x * rp;
    }
}

__global__ __launch_bounds__(kSampleBlock) void sample_block_kernel(const float* values, int n, float temperature,
                                                                    int k, uint64_t* lists)
{
    __shared__ uint64_t key[kSampleSlice];
    const int base = blockIdx.x * kSampleSlice;
    for (int j = threadIdx.x; j < kSampleSlice; j += kSampleBlock) {
        const int i = base + j;
        key[j] = i < n ? sample_key(values[i] / temperature, i) : ~uint64_t(0);
    }
    __syncthreads();
    bitonic_sort(key);
    for (int j = threadIdx.x; j < k; j += kSampleBlock) lists[size_t(blockIdx.x) * k + j] = key[j];
}

// Block b joins lists [b*group, min((b+1)*group, nlists)) of k keys each.
__global__ __launch_bounds__(kSampleBlock) void sample_merge_kernel(const uint64_t* src, int nlists, int k, int group,
                                                                    uint64_t* dst)
{
    __shared__ uint64_t key[kSampleSlice];
    const int first = blockIdx.x * group;
    const int count = (nlists - first < group ? nlists - first : group) * k;
    const uint64_t* in = src + size_t(first) * k;
    for (int j = threadIdx.x; j < kSampleSlice; j += kSampleBlock) key[j] = j < count ? in[j] : ~uint64_t(0);
    __syncthreads();
    bitonic_sort(key);
    for (int j = threadIdx.x; j < k; j += kSampleBlock) dst[size_t(blockIdx.x) * k + j] = key[j];
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

__global__ __launch_bounds__(kSampleFinish) void sample_finish_kernel(const float* values, float temperature,
                                                                      const uint64_t* list, int k, float top_p,
                                                                      const double* u, int32_t* out_token,
                                                                      int32_t* ids_out, float* probs_out)
{
    __shared__ int ids[kSampleMaxK];
    __shared__ float p[kSampleMaxK];
    __shared__ float drop[kSampleMaxK];
    __shared__ float total;
    const int t = threadIdx.x;
    // the k best values, recomputed exactly as the slice kernel computed them
    const float top = values[int(uint32_t(list[0]))] / temperature;
    for (int i = t; i < k; i += kSampleFinish) {
        const int id = int(uint32_t(list[i]));
        ids[i] = id;
        p[i] = spec_expf(values[id] / temperature - top);
    }
    __syncthreads();
    if (t == 0) total = pairwise_sum_f32(p, k);
    __syncthreads();
    for (int i = t; i < k; i += kSampleFinish) p[i] = p[i] / total;
    __syncthreads();
    if (top_p < 1.0f) {
        if (t == 0) {
            float c = 0.0f;
            for (int i = 0; i < k; ++i) {
                c = c + p[i];
                drop[i] = c - p[i];
            }
        }
        __syncthreads();
        for (int i = t; i < k; i += kSampleFinish)
            if (drop[i] >= top_p) p[i] = 0.0f;
        __syncthreads();
        if (t == 0) total = pairwise_sum_f32(p, k);
        __syncthreads();
        for (int i = t; i < k; i += kSampleFinish) p[i] = p[i] / total;
        __syncthreads();
    }
    if (t == 0) {
        // Generator.choice: cdf = cumsum(double(p)) / its last entry, the
        // token is ids[#{i : cdf_i <= u}]
        double last = 0.0;
        for (int i = 0; i < k; ++i) last = last + double(p[i]);
        const double draw = *u;
        double cdf = 0.0;
        int index = 0;
        for (int i = 0; i < k; ++i) {
            cdf = cdf + double(p[i]);
            if (cdf / last <= draw) index = i + 1;
        }
        if (index >= k) index = k - 1;
        *out_token = ids[index];
    }
    if (ids_out)
        for (int i = t; i < k; i += kSampleFinish) ids_out[i] = ids[i];
    if (probs_out)
        for (int i = t; i < k; i += kSampleFinish) probs_out[i] = p[i];
}

static size_t al256s(size_t v) { return (v + 255) & ~size_t(255); }

static int sample_slices(int n) { return (n + kSampleSlice - 1) / kSampleSlice; }

}  // namespace hq

using namespace hq;

extern "C" size_t hq_sample_workspace_bytes(int n, int top_k)
{
    if (n <= 0 || top_k <= 0) return 0;
    const int k = top_k < n ? top_k : n;
    const size_t lists = al256s(size_t(sample_slices(n)) * size_t(k) * 8);
    return al256s(size_t(n) * 4) + 2 * lists;
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
    const int k = top_k < n ? top_k : n;
    int nlists = sample_slices(n);
    hipStream_t s = static_cast<hipStream_t>(stream);
    char* ws = static_cast<char*>(workspace);
    float* values = reinterpret_cast<float*>(ws);
    const size_t list_bytes = al256s(size_t(nlists) * size_t(k) * 8);
    uint64_t* a = reinterpret_cast<uint64_t*>(ws + al256s(size_t(n) * 4));
    uint64_t* b = reinterpret_cast<uint64_t*>(ws + al256s(size_t(n) * 4) + list_bytes);
    const int cb = (n + kBlock - 1) / kBlock;
    hipLaunchKernelGGL(sample_copy_kernel, dim3(cb < 1024 ? cb : 1024), dim3(kBlock), 0, s, logits, n, values);
    if (repetition_penalty != 1.0f && n_generated > 0) {
        const int gb = (n_generated + kBlock - 1) / kBlock;
        hipLaunchKernelGGL(sample_penalty_kernel, dim3(gb < 64 ? gb : 64), dim3(kBlock), 0, s, logits, n, generated,
                           n_generated, repetition_penalty, values);
    }
    hipLaunchKernelGGL(sample_block_kernel, dim3(nlists), dim3(kSampleBlock), 0, s, values, n, temperature, k, a);
    const int group = kSampleSlice / k;       // >= 2 since k <= kSampleMaxK
    while (nlists > 1) {
        const int next = (nlists + group - 1) / group;
        hipLaunchKernelGGL(sample_merge_kernel, dim3(next), dim3(kSampleBlock), 0, s, a, nlists, k, group, b);
        uint64_t* swap = a;
        a = b;
        b = swap;
        nlists = next;
    }
    hipLaunchKernelGGL(sample_finish_kernel, dim3(1), dim3(kSampleFinish), 0, s, values, temperature, a, k, top_p, u,
                       out_token, ids_out, probs_out);
    return hipGetLastError() == hipSuccess ? HQ_OK : HQ_ERR_LAUNCH;
}
