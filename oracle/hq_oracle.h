/*
 * hq_oracle.h - CPU restatement of the Harsh4B int4 decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP
 * product path is compared against.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it; the product (harsh4b_amd)
 * never links, loads or calls it.
 *
 * Reference files restated (paths relative to the reference repository):
 *   cpu_kernels/litespark_int4.cpp   int4 x int8 GEMV (:22-76), GQA decode (:160-259)
 *   cpu_lightspark.py                pack (:139-146), state layout (:275-309),
 *                                    RoPE tables (:329-336), embedding (:341-349),
 *                                    projection (:351-371), qk-norm (:373-379),
 *                                    rope (:381-387), attention (:389-422),
 *                                    forward_token order (:424-468), argmax (:704-705),
 *                                    stochastic sampler (:706-726)
 *   MLX/bitnet_mlx.py:17-23          per-token absmax int8 quantization precedent
 *
 * The reference leaves the bits of several fp32 steps open (its kernels build
 * with -ffast-math and its quantizer / RMSNorm live in an absent third-party
 * wheel).  This file fixes them as the "hq numeric spec v1"; every function
 * header states the order of operations, and the HIP kernels follow the same
 * order so that results are bit-identical.
 *
 * Parity pins (tests/test_oracle_*.py): every function below is checked
 * against golden vectors, a float64 closed form, or brute force.  None is
 * "parity unpinned".
 */
#ifndef HQ_ORACLE_H
#define HQ_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar helpers of the spec ---- */
float or_expf(float x);
uint16_t or_f32_to_f16(float x);
float or_f16_to_f32(uint16_t h);
void or_f32_to_f16_array(const float* x, uint16_t* h, int64_t n);
void or_f16_to_f32_array(const uint16_t* h, float* x, int64_t n);

/* ---- packing ---- */
int or_pack_int4(const int8_t* w, int rows, int width, uint8_t* out);
int or_unpack_int4(const uint8_t* p, int rows, int width, int8_t* out);

/* ---- quantization, norms ---- */
float or_quantize_activation(const float* x, int n, int8_t* q);
void or_rmsnorm(const float* x, const float* gamma, float* y, int n, float eps);
void or_head_norm(float* x, const float* gamma, int heads, int head_dim, float eps);
void or_rope(float* x, int heads, int head_dim, const float* cos_row, const float* sin_row);

/* ---- GEMV ---- */
void or_int4_i8_gemv(const int8_t* x, const uint8_t* weights, const float* scales,
                     float activation_scale, float* output, int rows, int width);
/* Vector path control (AVX-512 VNNI where the CPU has it; same integers)
 * and OpenMP thread count of the GEMVs. */
void or_set_simd(int on);
int or_simd_active(void);
void or_set_threads(int n);
int or_max_threads(void);
void or_int4_i8_gemv_acc(const int8_t* x, const uint8_t* weights, int rows, int width,
                         int32_t* acc);
void or_int4_i8_gemm_acc(const int8_t* x, const uint8_t* weights, int m, int rows,
                         int width, int32_t* acc);
float or_quant_int4_gemv(const float* x, const uint8_t* weights, const float* scales,
                         float* output, int rows, int width, int8_t* q_out, int32_t* acc_out);

/* ---- attention ---- */
void or_gqa_decode_ref(const float* query, const float* keys, const float* values,
                       float* scores, float* output, int context, int kv_heads,
                       int groups, int head_dim, int score_stride);
void or_gqa_decode_split(const float* query, const uint16_t* keys, const uint16_t* values,
                         float* output, int context, int kv_heads, int groups,
                         int head_dim, int64_t time_stride, int chunk);
void or_gqa_decode_split_f32(const float* query, const float* keys, const float* values,
                             float* output, int context, int kv_heads, int groups,
                             int head_dim, int64_t time_stride, int chunk);

/* ---- SwiGLU, argmax ---- */
void or_swiglu(const float* gate, const float* up, float* out, int n);
int64_t or_argmax(const float* x, int64_t n);

/* ---- stochastic sampler (cpu_lightspark.py:706-726) ---- */
float or_pairwise_sum_f32(const float* a, int n);
int64_t or_sample_token(const float* logits, int64_t n, const int32_t* generated, int n_generated,
                        float repetition_penalty, float temperature, int top_k, float top_p, double u,
                        int32_t* ids_out, float* probs_out);

/* ---- full decode step ---- */
typedef struct or_layer {
    const uint8_t* qkv;      const float* qkv_scales;
    const uint8_t* o;        const float* o_scales;
    const uint8_t* gate_up;  const float* gate_up_scales;
    const uint8_t* down;     const float* down_scales;
    const float* input_norm; const float* post_norm;
    const float* q_norm;     const float* k_norm;
} or_layer;

typedef struct or_model {
    int32_t layers, hidden, intermediate, heads, kv_heads, head_dim, vocab, rope_positions;
    float eps;
    int32_t chunk;                 /* attention split length */
    const or_layer* layer;         /* [layers] */
    const uint8_t* embedding;      /* [vocab, hidden/2] */
    const float* embedding_scales; /* [vocab] */
    const float* final_norm;       /* [hidden] */
    const float* rope_cos;         /* [rope_positions, head_dim/2] */
    const float* rope_sin;
} or_model;

typedef struct or_state {
    int32_t capacity;
    int32_t position;
    int32_t kv_f32;    /* 0: fp16 cache (uint16 bits), 1: fp32 cache */
    int32_t pad;
    void* keys;        /* [layers, capacity, kv_heads, head_dim] */
    void* values;
    float* x;          /* [hidden] residual stream */
    float* logits;     /* [vocab] */
    float* trace;      /* nullable: [layers, hidden] residual after each layer */
} or_state;

void or_embedding(const or_model* m, int token, float* out);
int or_forward_token(const or_model* m, or_state* s, int token);

#ifdef __cplusplus
}
#endif
#endif
