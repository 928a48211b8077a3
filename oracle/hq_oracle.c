/*
 * hq_oracle.c - CPU restatement of the Harsh4B int4 decode path
 * (hq numeric spec v1).
 *
 * TEST INFRASTRUCTURE ONLY: the checker the HIP product is compared with.
 * It is loaded by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg, never by the product package.
 *
 * Build: oracle/Makefile (gcc, -O3 -ffp-contract=off, no -ffast-math, OpenMP).
 * Contraction is off so that every "a * b + c" below is two roundings unless
 * it is written as fmaf(); the HIP kernels are compiled the same way.
 *
 * Reference citations are file:line in the reference repository.
 */
#include "hq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>
#if defined(__x86_64__)
#include <immintrin.h>
#endif

/* ------------------------------------------------------------------------ */
/* bit helpers                                                               */
/* ------------------------------------------------------------------------ */
static inline float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* 2^k for k in [-126, 127] built from the exponent field. */
static inline float pow2i(int k) { return bits_to_f32((uint32_t)(k + 127) << 23); }

/*
 * exp(x) in fp32, the one implementation shared by softmax and SiLU.
 * Method: Cody & Waite argument reduction (W. J. Cody, W. Waite, "Software
 * Manual for the Elementary Functions", 1980): n = rint(x*log2(e)),
 * r = x - n*ln2 evaluated with a two-part ln2 (hi has 8 trailing zero bits)
 * through fmaf, then the degree-7 Taylor polynomial of e^r in Horner form
 * (|r| <= 0.347, truncation error < 2^-27 relative), then scaling by
 * 2^n split into two exact power-of-two multiplies.  Inputs below -87 give
 * exactly 0 (so no subnormal results ever occur) and inputs above
 * ln(FLT_MAX) give +inf.  Every operation is a single IEEE fp32 operation,
 * so the GPU reproduces it bit for bit.
 * Used in place of std::exp at litespark_int4.cpp:216 and np.exp at
 * cpu_lightspark.py:452.
 */
float or_expf(float x)
{
    if (x != x) return x;
    if (x > 0x1.62e430p+6f) return INFINITY;   /* 88.72284 */
    if (x < -87.0f) return 0.0f;
    const float n = rintf(x * 0x1.715476p+0f);  /* log2(e) */
    float r = fmaf(-n, 0x1.62e400p-1f, x);       /* ln2 hi = 0.693145751953125 */
    r = fmaf(-n, 0x1.7f7d1cp-20f, r);            /* ln2 lo = ln2 - hi */
    float p = 0x1.a01a02p-13f;                   /* 1/7! */
    p = fmaf(p, r, 0x1.6c16c2p-10f);             /* 1/6! */
    p = fmaf(p, r, 0x1.111112p-7f);              /* 1/5! */
    p = fmaf(p, r, 0x1.555556p-5f);              /* 1/4! */
    p = fmaf(p, r, 0x1.555556p-3f);              /* 1/3! */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const int ni = (int)n;
    const int n1 = ni / 2;
    const int n2 = ni - n1;
    p = p * pow2i(n1);
    p = p * pow2i(n2);
    return p;
}

/*
 * fp32 -> fp16 bits, IEEE round-to-nearest-even (the KV cache format).
 * Normal range: round at mantissa bit 13 with the ties-to-even carry; the
 * carry may move the value into the next binade or to infinity, both of
 * which are the correctly rounded result.  Below 2^-14 the half value is an
 * integer multiple of 2^-24, so a*2^24 (exact) is rounded with rintf.
 */
uint16_t or_f32_to_f16(float f)
{
    const uint32_t x = f32_to_bits(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x1FFu));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);   /* >= 65520 -> inf */
    if (ax < 0x38800000u) {                                      /* < 2^-14 */
        const float a = bits_to_f32(ax);
        return (uint16_t)(sign | (uint16_t)rintf(a * 16777216.0f));
    }
    const uint32_t rounded = ax + 0xFFFu + ((ax >> 13) & 1u);
    return (uint16_t)(sign | ((rounded - 0x38000000u) >> 13));
}

float or_f16_to_f32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    if (e == 0) {
        const float v = (float)m * 0x1p-24f;
        return sign ? -v : v;
    }
    if (e == 31) return bits_to_f32(sign | 0x7F800000u | (m << 13));
    return bits_to_f32(sign | ((e + 112u) << 23) | (m << 13));
}

void or_f32_to_f16_array(const float* x, uint16_t* h, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) h[i] = or_f32_to_f16(x[i]);
}

void or_f16_to_f32_array(const uint16_t* h, float* x, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) x[i] = or_f16_to_f32(h[i]);
}

/* ------------------------------------------------------------------------ */
/* packing and unpacking                                                    */
/* ------------------------------------------------------------------------ */
/*
 * cpu_lightspark.py:139-146 (_pack_int4): P[n,j] = (W[n,2j] & 0xF) |
 * ((W[n,2j+1] & 0xF) << 4).  Returns -1 when a value is outside [-7,7]
 * (:143-144) and -2 for an odd width (:141-142), writing nothing.
 */
int or_pack_int4(const int8_t* w, int rows, int width, uint8_t* out)
{
    if (width % 2) return -2;
    const int64_t total = (int64_t)rows * width;
    for (int64_t i = 0; i < total; ++i)
        if (w[i] < -7 || w[i] > 7) return -1;
    const int half = width / 2;
    for (int r = 0; r < rows; ++r)
        for (int j = 0; j < half; ++j) {
            const uint8_t lo = (uint8_t)w[(int64_t)r * width + 2 * j] & 0xFu;
            const uint8_t hi = (uint8_t)w[(int64_t)r * width + 2 * j + 1] & 0xFu;
            out[(int64_t)r * half + j] = (uint8_t)(lo | (hi << 4));
        }
    return 0;
}

/* litespark_int4.cpp:66-68: low = (int8)(b << 4) >> 4, high = (int8)b >> 4. */
static inline int nib_lo(uint8_t b) { return (int)(int8_t)(uint8_t)(b << 4) >> 4; }
static inline int nib_hi(uint8_t b) { return (int)((int8_t)b) >> 4; }

int or_unpack_int4(const uint8_t* p, int rows, int width, int8_t* out)
{
    if (width % 2) return -2;
    const int half = width / 2;
    for (int r = 0; r < rows; ++r)
        for (int j = 0; j < half; ++j) {
            const uint8_t b = p[(int64_t)r * half + j];
            out[(int64_t)r * width + 2 * j] = (int8_t)nib_lo(b);
            out[(int64_t)r * width + 2 * j + 1] = (int8_t)nib_hi(b);
        }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* per-token int8 activation quantization                                    */
/* ------------------------------------------------------------------------ */
/*
 * Stands in for the third-party kernel.quantize_activation called at
 * cpu_lightspark.py:433,443,449,457,463 (whose source is not in the
 * reference).  Symmetric absmax as in MLX/bitnet_mlx.py:17-23:
 *   amax = max(max_i |x_i|, 1e-5);  inv = 127 / amax;
 *   q_i = clamp(rint(x_i * inv), -127, 127)   (round half to even)
 * and returns the dequantization multiplier amax / 127, which the GEMV
 * epilogue multiplies by (litespark_int4.cpp:73-74).
 */
float or_quantize_activation(const float* x, int n, int8_t* q)
{
    float amax = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    amax = fmaxf(amax, 1e-5f);
    const float inv = 127.0f / amax;
    for (int i = 0; i < n; ++i) {
        float v = rintf(x[i] * inv);
        if (v > 127.0f) v = 127.0f;
        if (v < -127.0f) v = -127.0f;
        q[i] = (int8_t)v;
    }
    return amax / 127.0f;
}

/* ------------------------------------------------------------------------ */
/* RMSNorm and per-head norm                                                 */
/* ------------------------------------------------------------------------ */
/*
 * Sum of squares with the spec's fixed tree: lane l of `lanes` accumulates
 * x[l], x[l+lanes], ... with fmaf in ascending order from 0, then the lanes
 * are folded by halving: v[i] += v[i+o] for o = lanes/2 ... 1.
 */
static float tree_sum_sq(const float* x, int n, int lanes)
{
    float v[256];
    for (int l = 0; l < lanes; ++l) {
        float p = 0.0f;
        for (int i = l; i < n; i += lanes) p = fmaf(x[i], x[i], p);
        v[l] = p;
    }
    for (int o = lanes / 2; o >= 1; o >>= 1)
        for (int l = 0; l < o; ++l) v[l] = v[l] + v[l + o];
    return v[0];
}

/*
 * RMSNorm over the hidden vector, standing in for the third-party
 * kernel.rmsnorm_into (cpu_lightspark.py:431,447,461).  The operation order
 * is the one _qk_norm uses (cpu_lightspark.py:374-379):
 *   ss = sum x^2 (256-lane tree); r = sqrt(ss / n + eps); y = (x / r) * gamma
 */
void or_rmsnorm(const float* x, const float* gamma, float* y, int n, float eps)
{
    const float ss = tree_sum_sq(x, n, 256);
    const float ms = ss / (float)n;
    const float r = sqrtf(ms + eps);
    for (int i = 0; i < n; ++i) y[i] = (x[i] / r) * gamma[i];
}

/* cpu_lightspark.py:373-379 (_qk_norm), per head, 64-lane tree, in place. */
void or_head_norm(float* x, const float* gamma, int heads, int head_dim, float eps)
{
    for (int h = 0; h < heads; ++h) {
        float* v = x + (int64_t)h * head_dim;
        const float ss = tree_sum_sq(v, head_dim, 64);
        const float ms = ss / (float)head_dim;
        const float r = sqrtf(ms + eps);
        for (int i = 0; i < head_dim; ++i) v[i] = (v[i] / r) * gamma[i];
    }
}

/*
 * cpu_lightspark.py:381-387 (_rope), half-split rotation with the host
 * tables of :329-336:  a' = a*c - b*s,  b' = b*c + a*s  (a = x[i],
 * b = x[i + d/2]); each product is rounded before the add.
 */
void or_rope(float* x, int heads, int head_dim, const float* cos_row, const float* sin_row)
{
    const int half = head_dim / 2;
    for (int h = 0; h < heads; ++h) {
        float* v = x + (int64_t)h * head_dim;
        for (int i = 0; i < half; ++i) {
            const float a = v[i], b = v[i + half];
            const float c = cos_row[i], s = sin_row[i];
            const float ac = a * c, bs = b * s, bc = b * c, as = a * s;
            v[i] = ac - bs;
            v[i + half] = bc + as;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* packed int4 x int8 GEMV                                                   */
/* ------------------------------------------------------------------------ */
/*
 * litespark_int4.cpp:22-76.  acc = sum_k W[n,k] * x[k] in int32 (the NEON
 * body and the scalar tail compute the same integer), then
 * out = ((float)acc * activation_scale) * scale[n] (:73-74).
 *
 * Two implementations of the same integer: the scalar loop, and on x86 CPUs
 * with AVX-512 VNNI an SDOT-like path (the reference's NEON SDOT role, done
 * with vpdpbusd): the activations are split once per call into even and
 * odd elements (the low and high nibbles' partners); each 64-byte block of
 * a row gives its 64 low and 64 high nibbles as unsigned u = w + 8 in
 * [0, 15], vpdpbusd accumulates u * x in int32, and
 * sum(w * x) = sum(u * x) - 8 * sum(x) exactly (no term can overflow:
 * |u * x| <= 15 * 128).  or_set_simd(0) forces the scalar loop, which
 * tests compare with the vector path.
 */
static int g_simd = 1;

void or_set_simd(int on) { g_simd = on != 0; }

int or_simd_active(void)
{
#if defined(__x86_64__)
    return g_simd && __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512vnni");
#else
    return 0;
#endif
}

void or_set_threads(int n)
{
    if (n > 0) omp_set_num_threads(n);
}

int or_max_threads(void) { return omp_get_max_threads(); }

static void gemv_acc_scalar(const int8_t* x, const uint8_t* weights, int rows, int width, int32_t* acc)
{
    const int half = width >> 1;
#pragma omp parallel for schedule(static) if (rows >= 64)
    for (int r = 0; r < rows; ++r) {
        const uint8_t* row = weights + (int64_t)r * half;
        int32_t s = 0;
        for (int j = 0; j < half; ++j) {
            const uint8_t b = row[j];
            s += nib_lo(b) * (int32_t)x[2 * j] + nib_hi(b) * (int32_t)x[2 * j + 1];
        }
        acc[r] = s;
    }
}

#if defined(__x86_64__)
__attribute__((target("avx512f,avx512bw,avx512vnni")))
static void gemv_acc_vnni(const int8_t* x, const uint8_t* weights, int rows, int width, int32_t* acc)
{
    const int half = width >> 1;
    const int body = half & ~63;          /* packed bytes in whole 64-byte blocks */
    int8_t* xe = (int8_t*)malloc((size_t)(half > 0 ? half : 1));
    int8_t* xo = (int8_t*)malloc((size_t)(half > 0 ? half : 1));
    int32_t xsum = 0;                      /* sum of the activations the blocks cover */
    for (int j = 0; j < half; ++j) {
        xe[j] = x[2 * j];
        xo[j] = x[2 * j + 1];
        if (j < body) xsum += (int32_t)x[2 * j] + (int32_t)x[2 * j + 1];
    }
    const __m512i lo_mask = _mm512_set1_epi8(0x0F);
    const __m512i bias = _mm512_set1_epi8(0x08);
#pragma omp parallel for schedule(static) if (rows >= 64)
    for (int r = 0; r < rows; ++r) {
        const uint8_t* row = weights + (int64_t)r * half;
        __m512i a0 = _mm512_setzero_si512(), a1 = _mm512_setzero_si512();
        for (int j = 0; j < body; j += 64) {
            const __m512i w = _mm512_loadu_si512((const void*)(row + j));
            const __m512i lo = _mm512_xor_si512(_mm512_and_si512(w, lo_mask), bias);
            const __m512i hi = _mm512_xor_si512(_mm512_and_si512(_mm512_srli_epi16(w, 4), lo_mask), bias);
            a0 = _mm512_dpbusd_epi32(a0, lo, _mm512_loadu_si512((const void*)(xe + j)));
            a1 = _mm512_dpbusd_epi32(a1, hi, _mm512_loadu_si512((const void*)(xo + j)));
        }
        int32_t s = _mm512_reduce_add_epi32(_mm512_add_epi32(a0, a1)) - 8 * xsum;
        for (int j = body; j < half; ++j) {
            const uint8_t b = row[j];
            s += nib_lo(b) * (int32_t)xe[j] + nib_hi(b) * (int32_t)xo[j];
        }
        acc[r] = s;
    }
    free(xe);
    free(xo);
}
#endif

void or_int4_i8_gemv_acc(const int8_t* x, const uint8_t* weights, int rows, int width,
                         int32_t* acc)
{
#if defined(__x86_64__)
    if (or_simd_active()) {
        gemv_acc_vnni(x, weights, rows, width, acc);
        return;
    }
#endif
    gemv_acc_scalar(x, weights, rows, width, acc);
}

void or_int4_i8_gemv(const int8_t* x, const uint8_t* weights, const float* scales,
                     float activation_scale, float* output, int rows, int width)
{
    int32_t* acc = (int32_t*)malloc(sizeof(int32_t) * (size_t)(rows > 0 ? rows : 1));
    or_int4_i8_gemv_acc(x, weights, rows, width, acc);
    for (int r = 0; r < rows; ++r)
        output[r] = ((float)acc[r] * activation_scale) * scales[r];
    free(acc);
}

/* Batched form (config 4): m independent GEMVs sharing the weights. */
void or_int4_i8_gemm_acc(const int8_t* x, const uint8_t* weights, int m, int rows,
                         int width, int32_t* acc)
{
    for (int i = 0; i < m; ++i)
        or_int4_i8_gemv_acc(x + (int64_t)i * width, weights, rows, width,
                            acc + (int64_t)i * rows);
}

/* Quantization + GEMV as one call: the fused hot-path entry.  Returns act_scale. */
float or_quant_int4_gemv(const float* x, const uint8_t* weights, const float* scales,
                         float* output, int rows, int width, int8_t* q_out, int32_t* acc_out)
{
    int8_t* q = q_out ? q_out : (int8_t*)malloc((size_t)width);
    int32_t* acc = acc_out ? acc_out : (int32_t*)malloc(sizeof(int32_t) * (size_t)rows);
    const float act = or_quantize_activation(x, width, q);
    or_int4_i8_gemv_acc(q, weights, rows, width, acc);
    for (int r = 0; r < rows; ++r) output[r] = ((float)acc[r] * act) * scales[r];
    if (!q_out) free(q);
    if (!acc_out) free(acc);
    return act;
}

/* ------------------------------------------------------------------------ */
/* GQA decode attention                                                      */
/* ------------------------------------------------------------------------ */
/*
 * Literal restatement of litespark_gqa_decode (litespark_int4.cpp:160-259)
 * with fp32 keys/values in its [time, kv_head, head_dim] layout: four
 * 4-wide partial FMA accumulators over 16-dim blocks, combined as the
 * vector adds at :204-206 and a pairwise horizontal add; sequential max,
 * std::exp, sequential denominator, one reciprocal, then per-dim FMA
 * accumulation over time.  The reference builds with -ffast-math, so this
 * is the algorithm, not its exact bits; it is used with a tolerance.
 */
void or_gqa_decode_ref(const float* query, const float* keys, const float* values,
                       float* scores, float* output, int context, int kv_heads,
                       int groups, int head_dim, int score_stride)
{
    const int query_heads = kv_heads * groups;
    const int kv_time_stride = kv_heads * head_dim;
    const float scale = 1.0f / sqrtf((float)head_dim);
    for (int qh = 0; qh < query_heads; ++qh) {
        const int kvh = qh / groups;
        const float* q = query + (int64_t)qh * head_dim;
        float* score = scores + (int64_t)qh * score_stride;
        float maximum = -3.402823466e38f;
        for (int t = 0; t < context; ++t) {
            const float* key = keys + (int64_t)t * kv_time_stride + (int64_t)kvh * head_dim;
            float s[4][4] = {{0}};
            int d = 0;
            for (; d + 16 <= head_dim; d += 16)
                for (int v = 0; v < 4; ++v)
                    for (int j = 0; j < 4; ++j)
                        s[v][j] = fmaf(q[d + 4 * v + j], key[d + 4 * v + j], s[v][j]);
            float lanes[4];
            for (int j = 0; j < 4; ++j) lanes[j] = (s[0][j] + s[1][j]) + (s[2][j] + s[3][j]);
            float dot = (lanes[0] + lanes[1]) + (lanes[2] + lanes[3]);
            for (; d < head_dim; ++d) dot += q[d] * key[d];
            score[t] = dot * scale;
            if (score[t] > maximum) maximum = score[t];
        }
        float denominator = 0.0f;
        for (int t = 0; t < context; ++t) {
            const float p = expf(score[t] - maximum);
            score[t] = p;
            denominator += p;
        }
        const float inv = 1.0f / denominator;
        for (int t = 0; t < context; ++t) score[t] *= inv;
        float* out = output + (int64_t)qh * head_dim;
        for (int d = 0; d < head_dim; ++d) {
            float acc = 0.0f;
            for (int t = 0; t < context; ++t)
                acc = fmaf(values[(int64_t)t * kv_time_stride + (int64_t)kvh * head_dim + d],
                           score[t], acc);
            out[d] = acc;
        }
    }
}

/*
 * The spec order of the fused HIP attention (same math as :160-259, split
 * along time so that the work fills the GPU).  fp16 keys/values, element
 * (t, kv_head, d) at t*time_stride + kv_head*head_dim + d.
 *   score:  16 partial dots, partial l covering dims [l*D/16, (l+1)*D/16)
 *           with fmaf ascending from 0, halving tree over the 16 partials,
 *           then dot * (1/sqrt(D)).
 *   chunk c (positions [c*chunk, c*chunk+chunk) below context):
 *           m_c = max score; e_t = exp(s_t - m_c); l_c = halving tree over
 *           the `chunk` slots (empty slots hold 0); o_c[d] = fmaf chain of
 *           e_t * v_t[d] over ascending t.
 *   combine: M = max m_c; for c ascending a = exp(m_c - M),
 *           L = fmaf(a, l_c, L), O[d] = fmaf(a, o_c[d], O[d]);
 *           out[d] = O[d] * (1 / L)   (the reciprocal of :220-222).
 * chunk must be a power of two <= 256; head_dim a multiple of 16, <= 256.
 */
static inline float kv_load(const void* base, int f32, int64_t i)
{
    return f32 ? ((const float*)base)[i] : or_f16_to_f32(((const uint16_t*)base)[i]);
}

static void gqa_split_impl(const float* query, const void* keys, const void* values, int kv_f32,
                           float* output, int context, int kv_heads, int groups,
                           int head_dim, int64_t time_stride, int chunk)
{
    const float scale = 1.0f / sqrtf((float)head_dim);
    const int nchunks = (context + chunk - 1) / chunk;
    const int dpl = head_dim / 16;
    /* query heads are independent: one OpenMP thread per head at a time
     * (from 32 positions up: below that a head is too little work) */
#pragma omp parallel for schedule(dynamic, 1) if (context >= 32)
    for (int qh = 0; qh < kv_heads * groups; ++qh) {
        {
            const int g = qh / groups;
            float* m = (float*)malloc(sizeof(float) * (size_t)nchunks);
            float* l = (float*)malloc(sizeof(float) * (size_t)nchunks);
            float* o = (float*)malloc(sizeof(float) * (size_t)nchunks * (size_t)head_dim);
            float s[256], e[256], tree[256], kf[256];
            const float* q = query + (int64_t)qh * head_dim;
            for (int c = 0; c < nchunks; ++c) {
                float mc = -INFINITY;
                for (int i = 0; i < chunk; ++i) {
                    const int t = c * chunk + i;
                    if (t >= context) { s[i] = -INFINITY; continue; }
                    const int64_t kb = (int64_t)t * time_stride + (int64_t)g * head_dim;
                    for (int d = 0; d < head_dim; ++d) kf[d] = kv_load(keys, kv_f32, kb + d);
                    float part[16];
                    for (int ln = 0; ln < 16; ++ln) {
                        float p = 0.0f;
                        for (int j = 0; j < dpl; ++j) {
                            const int d = ln * dpl + j;
                            p = fmaf(q[d], kf[d], p);
                        }
                        part[ln] = p;
                    }
                    for (int off = 8; off >= 1; off >>= 1)
                        for (int ln = 0; ln < off; ++ln) part[ln] = part[ln] + part[ln + off];
                    s[i] = part[0] * scale;
                    if (s[i] > mc) mc = s[i];
                }
                for (int i = 0; i < chunk; ++i) {
                    const int t = c * chunk + i;
                    e[i] = (t < context) ? or_expf(s[i] - mc) : 0.0f;
                    tree[i] = e[i];
                }
                for (int off = chunk / 2; off >= 1; off >>= 1)
                    for (int i = 0; i < off; ++i) tree[i] = tree[i] + tree[i + off];
                m[c] = mc;
                l[c] = tree[0];
                for (int d = 0; d < head_dim; ++d) {
                    float acc = 0.0f;
                    for (int i = 0; i < chunk; ++i) {
                        const int t = c * chunk + i;
                        if (t >= context) break;
                        const float v = kv_load(
                            values, kv_f32, (int64_t)t * time_stride + (int64_t)g * head_dim + d);
                        acc = fmaf(e[i], v, acc);
                    }
                    o[(int64_t)c * head_dim + d] = acc;
                }
            }
            float M = -INFINITY;
            for (int c = 0; c < nchunks; ++c) if (m[c] > M) M = m[c];
            float L = 0.0f;
            float* out = output + (int64_t)qh * head_dim;
            for (int d = 0; d < head_dim; ++d) out[d] = 0.0f;
            for (int c = 0; c < nchunks; ++c) {
                const float a = or_expf(m[c] - M);
                L = fmaf(a, l[c], L);
                for (int d = 0; d < head_dim; ++d)
                    out[d] = fmaf(a, o[(int64_t)c * head_dim + d], out[d]);
            }
            const float inv = 1.0f / L;
            for (int d = 0; d < head_dim; ++d) out[d] = out[d] * inv;
            free(m); free(l); free(o);
        }
    }
}

void or_gqa_decode_split(const float* query, const uint16_t* keys, const uint16_t* values,
                         float* output, int context, int kv_heads, int groups,
                         int head_dim, int64_t time_stride, int chunk)
{
    gqa_split_impl(query, keys, values, 0, output, context, kv_heads, groups, head_dim,
                   time_stride, chunk);
}

void or_gqa_decode_split_f32(const float* query, const float* keys, const float* values,
                             float* output, int context, int kv_heads, int groups,
                             int head_dim, int64_t time_stride, int chunk)
{
    gqa_split_impl(query, keys, values, 1, output, context, kv_heads, groups, head_dim,
                   time_stride, chunk);
}

/* ------------------------------------------------------------------------ */
/* SwiGLU, argmax                                                            */
/* ------------------------------------------------------------------------ */
/* cpu_lightspark.py:451-455: negate, exp, +1, divide, multiply. */
void or_swiglu(const float* gate, const float* up, float* out, int n)
{
    for (int i = 0; i < n; ++i) {
        const float t = 1.0f + or_expf(-gate[i]);
        out[i] = (gate[i] / t) * up[i];
    }
}

/*
 * cpu_lightspark.py:704-705: int(np.argmax(logits)); the first maximal
 * index wins, and (as numpy does) the first NaN wins over any number.
 */
int64_t or_argmax(const float* x, int64_t n)
{
    int64_t best = 0;
    for (int64_t i = 1; i < n; ++i) {
        const float a = x[i], b = x[best];
        if (b != b) break;
        if (a != a || a > b) best = i;
    }
    return best;
}

/* ------------------------------------------------------------------------ */
/* stochastic sampler                                                        */
/* ------------------------------------------------------------------------ */
/* numpy's float32 add.reduce order for n <= 128 (pairwise_sum): n < 8 a
 * sequential sum from 0; else eight strided accumulators, combined as
 * ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)), then the n % 8 tail added in order. */
float or_pairwise_sum_f32(const float* a, int n)
{
    /* numpy's pairwise_sum (umath loops_utils.h.src): < 8 values in order,
       <= 128 values in eight running sums, larger halves split at a
       multiple of 8 below n/2 */
    if (n < 8) {
        float r = 0.0f;
        for (int i = 0; i < n; ++i) r += a[i];
        return r;
    }
    if (n > 128) {
        int n2 = n / 2;
        n2 -= n2 % 8;
        return or_pairwise_sum_f32(a, n2) + or_pairwise_sum_f32(a + n2, n - n2);
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

/* Rank of a value: larger first, NaN after every number. */
static int or_sample_before(float a, int64_t ia, float b, int64_t ib)
{
    const int na = a != a, nb = b != b;
    if (na != nb) return nb;                 /* a number before a NaN */
    if (!na && a != b) return a > b;
    return ia < ib;                          /* equal values (or two NaNs): lower index */
}

/*
 * cpu_lightspark.py:706-726, with the repo's exp (or_expf) and the top-k order
 * among equal values fixed to ascending index (numpy leaves it open):
 *   v = logits (fp32); for each distinct id in generated, when rp != 1:
 *       v[id] = v[id] > 0 ? v[id] / rp : v[id] * rp
 *   v[i] = v[i] / temperature                      (every element)
 *   ids = the k = min(top_k, n) largest v, by value descending
 *   s_i = v[ids[i]] - v[ids[0]];  p_i = exp(s_i);  p_i = p_i / sum(p)
 *   if top_p < 1: c = cumsum(p) (fp32, in order); p_i = 0 where c_i - p_i >= top_p;
 *                 p_i = p_i / sum(p)
 *   Generator.choice(ids, p): cdf = cumsum((double)p); cdf_i = cdf_i / cdf_{k-1};
 *                 index = #{i : cdf_i <= u} with u = generator.random()
 * sums are or_pairwise_sum_f32 (numpy's order).  Writes the k ids and final
 * probabilities when ids_out / probs_out are given; returns the token.
 */
int64_t or_sample_token(const float* logits, int64_t n, const int32_t* generated, int n_generated,
                        float repetition_penalty, float temperature, int top_k, float top_p, double u,
                        int32_t* ids_out, float* probs_out)
{
    float* v = (float*)malloc((size_t)n * sizeof(float));
    for (int64_t i = 0; i < n; ++i) v[i] = logits[i];
    if (repetition_penalty != 1.0f)
        for (int g = 0; g < n_generated; ++g) {
            const int32_t id = generated[g];
            if (id < 0 || id >= n) continue;
            const float x = logits[id];
            v[id] = x > 0.0f ? x / repetition_penalty : x * repetition_penalty;
        }
    for (int64_t i = 0; i < n; ++i) v[i] = v[i] / temperature;
    int k = top_k < n ? top_k : (int)n;
    if (k < 1) k = 1;
    int64_t* ids = (int64_t*)malloc((size_t)k * sizeof(int64_t));
    int have = 0;
    for (int64_t i = 0; i < n; ++i) {
        if (have == k && !or_sample_before(v[i], i, v[ids[k - 1]], ids[k - 1])) continue;
        int pos = have < k ? have++ : k - 1;
        while (pos > 0 && or_sample_before(v[i], i, v[ids[pos - 1]], ids[pos - 1])) {
            ids[pos] = ids[pos - 1];
            --pos;
        }
        ids[pos] = i;
    }
    float* p = (float*)malloc((size_t)k * sizeof(float));
    const float top = v[ids[0]];
    for (int i = 0; i < k; ++i) p[i] = or_expf(v[ids[i]] - top);
    float s = or_pairwise_sum_f32(p, k);
    for (int i = 0; i < k; ++i) p[i] = p[i] / s;
    if (top_p < 1.0f) {
        float c = 0.0f;
        float* drop = (float*)malloc((size_t)k * sizeof(float));
        for (int i = 0; i < k; ++i) {
            c = c + p[i];
            drop[i] = c - p[i];
        }
        for (int i = 0; i < k; ++i)
            if (drop[i] >= top_p) p[i] = 0.0f;
        free(drop);
        s = or_pairwise_sum_f32(p, k);
        for (int i = 0; i < k; ++i) p[i] = p[i] / s;
    }
    double* cdf = (double*)malloc((size_t)k * sizeof(double));
    double c = 0.0;
    for (int i = 0; i < k; ++i) {
        c = c + (double)p[i];
        cdf[i] = c;
    }
    const double last = cdf[k - 1];
    int index = 0;
    for (int i = 0; i < k; ++i) {
        cdf[i] = cdf[i] / last;
        if (cdf[i] <= u) index = i + 1;
    }
    if (index >= k) index = k - 1;
    const int64_t token = ids[index];
    if (ids_out)
        for (int i = 0; i < k; ++i) ids_out[i] = (int32_t)ids[i];
    if (probs_out)
        for (int i = 0; i < k; ++i) probs_out[i] = p[i];
    free(cdf); free(p); free(ids); free(v);
    return token;
}

/* ------------------------------------------------------------------------ */
/* embedding, forward_token                                                   */
/* ------------------------------------------------------------------------ */
/* cpu_lightspark.py:341-349: decode one int4 row, multiply by its scale. */
void or_embedding(const or_model* m, int token, float* out)
{
    const int half = m->hidden / 2;
    const uint8_t* row = m->embedding + (int64_t)token * half;
    const float s = m->embedding_scales[token];
    for (int j = 0; j < half; ++j) {
        out[2 * j] = (float)nib_lo(row[j]) * s;
        out[2 * j + 1] = (float)nib_hi(row[j]) * s;
    }
}

static void projection(const float* values, int width, const uint8_t* w, const float* scales,
                       int rows, float* out, int8_t* q, int32_t* acc)
{
    const float act = or_quantize_activation(values, width, q);
    or_int4_i8_gemv_acc(q, w, rows, width, acc);
    for (int r = 0; r < rows; ++r) out[r] = ((float)acc[r] * act) * scales[r];
}

/*
 * One decode step in the order of cpu_lightspark.py:424-468, with the fp16
 * KV cache of the benchmark configurations (or, with kv_f32, the fp32 cache
 * of the reference's QwenDecodeState, :290-291) and the split attention.
 * Returns the greedy token (argmax of the logits), -1 when the state is full
 * (:426-427) and -2 for a token outside the vocabulary (:342-343).
 */
int or_forward_token(const or_model* m, or_state* st, int token)
{
    if (st->position >= st->capacity) return -1;
    if (token < 0 || token >= m->vocab) return -2;
    const int H = m->hidden, I = m->intermediate, D = m->head_dim;
    const int nq = m->heads, nkv = m->kv_heads, groups = nq / nkv;
    const int qsz = nq * D, kvsz = nkv * D;
    const int pos = st->position;
    const int64_t layer_stride = (int64_t)st->capacity * kvsz;
    const int wmax = I > qsz ? (I > H ? I : H) : (qsz > H ? qsz : H);

    float* normed = (float*)malloc(sizeof(float) * (size_t)H);
    float* qkv = (float*)malloc(sizeof(float) * (size_t)(qsz + 2 * kvsz));
    float* attended = (float*)malloc(sizeof(float) * (size_t)qsz);
    float* proj = (float*)malloc(sizeof(float) * (size_t)H);
    float* gate_up = (float*)malloc(sizeof(float) * (size_t)(2 * I));
    float* activated = (float*)malloc(sizeof(float) * (size_t)I);
    int8_t* q8 = (int8_t*)malloc((size_t)wmax);
    int32_t* acc = (int32_t*)malloc(sizeof(int32_t) * (size_t)(m->vocab > 2 * I ? m->vocab : 2 * I));
    float* x = st->x;

    or_embedding(m, token, x);
    for (int li = 0; li < m->layers; ++li) {
        const or_layer* L = &m->layer[li];
        or_rmsnorm(x, L->input_norm, normed, H, m->eps);
        projection(normed, H, L->qkv, L->qkv_scales, qsz + 2 * kvsz, qkv, q8, acc);
        float* q = qkv;
        float* k = qkv + qsz;
        float* v = qkv + qsz + kvsz;
        or_head_norm(q, L->q_norm, nq, D, m->eps);
        or_head_norm(k, L->k_norm, nkv, D, m->eps);
        const float* cr = m->rope_cos + (int64_t)pos * (D / 2);
        const float* sr = m->rope_sin + (int64_t)pos * (D / 2);
        or_rope(q, nq, D, cr, sr);
        or_rope(k, nkv, D, cr, sr);
        if (st->kv_f32) {
            float* kc = (float*)st->keys + li * layer_stride;
            float* vc = (float*)st->values + li * layer_stride;
            memcpy(kc + (int64_t)pos * kvsz, k, sizeof(float) * (size_t)kvsz);
            memcpy(vc + (int64_t)pos * kvsz, v, sizeof(float) * (size_t)kvsz);
            or_gqa_decode_split_f32(q, kc, vc, attended, pos + 1, nkv, groups, D, kvsz, m->chunk);
        } else {
            uint16_t* kc = (uint16_t*)st->keys + li * layer_stride;
            uint16_t* vc = (uint16_t*)st->values + li * layer_stride;
            or_f32_to_f16_array(k, kc + (int64_t)pos * kvsz, kvsz);
            or_f32_to_f16_array(v, vc + (int64_t)pos * kvsz, kvsz);
            or_gqa_decode_split(q, kc, vc, attended, pos + 1, nkv, groups, D, kvsz, m->chunk);
        }
        projection(attended, qsz, L->o, L->o_scales, H, proj, q8, acc);
        for (int i = 0; i < H; ++i) x[i] = x[i] + proj[i];
        or_rmsnorm(x, L->post_norm, normed, H, m->eps);
        projection(normed, H, L->gate_up, L->gate_up_scales, 2 * I, gate_up, q8, acc);
        or_swiglu(gate_up, gate_up + I, activated, I);
        projection(activated, I, L->down, L->down_scales, H, proj, q8, acc);
        for (int i = 0; i < H; ++i) x[i] = x[i] + proj[i];
        if (st->trace) memcpy(st->trace + (int64_t)li * H, x, sizeof(float) * (size_t)H);
    }
    or_rmsnorm(x, m->final_norm, normed, H, m->eps);
    projection(normed, H, m->embedding, m->embedding_scales, m->vocab, st->logits, q8, acc);
    st->position += 1;
    free(normed); free(qkv); free(attended); free(proj); free(gate_up); free(activated);
    free(q8); free(acc);
    return (int)or_argmax(st->logits, m->vocab);
}
