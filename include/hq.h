/*
 * hq.h - C ABI of libhq.so, the MI355X (gfx950) int4 decode hot path.
 *
 * Every entry point takes DEVICE pointers (HIP device memory, e.g. a
 * tensor's data_ptr()), plain sizes, and a HIP stream passed as `void*`
 * (NULL = the default stream).  Work is enqueued asynchronously on that
 * stream; nothing is allocated, freed or retained by the library.  Each call
 * returns HQ_OK or an HQ_ERR_* code; shapes are validated on the host before
 * any launch, so a bad call launches nothing.
 *
 * Reference citations are file:line in the reference repository
 * (OneBit-AI/Harsh4B).  The reference binds its native library through
 * ctypes with host pointers and no return value (cpu_lightspark.py:71-111);
 * this ABI keeps each function's argument order and meaning and adds the
 * stream and the status return.
 */
#ifndef HQ_H
#define HQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HQ_OK 0
#define HQ_ERR_ARG 1      /* bad shape, size or null pointer */
#define HQ_ERR_ALIGN 2    /* pointer alignment a kernel needs is not met */
#define HQ_ERR_LAUNCH 3   /* the HIP launch failed */
#define HQ_ERR_DEVICE 4   /* no usable gfx950 device */

/* Text for a status code (static storage). */
const char* hq_status_string(int status);
/* ABI version: 100 * major + minor. */
int hq_abi_version(void);

/* ----------------------------------------------------------- int4 GEMV --
 * Packed signed-int4 x int8 GEMV.  Replaces litespark_int4_i8_gemv,
 * _nopf, _pf256 and _pf512 (cpu_kernels/litespark_int4.cpp:78-108; the four
 * differ only in a CPU prefetch distance), bound at cpu_lightspark.py:71-93:
 *   output[n] = ((float)sum_k W[n,k] * x[k] * activation_scale) * scales[n]
 * x: int8 [width]; weights: uint8 [rows, width/2], two's-complement nibbles,
 * low nibble = even column (cpu_lightspark.py:139-146); scales: fp32 [rows];
 * output: fp32 [rows].  width must be even and <= 32768. */
int hq_int4_i8_gemv(const int8_t* x, const uint8_t* weights, const float* scales,
                    float activation_scale, float* output, int rows, int width,
                    void* stream);

/* ----------------------------------------------- quantization + GEMV --
 * The fused hot-path projection: per-token int8 quantization of fp32 x
 * (replaces the third-party kernel.quantize_activation called at
 * cpu_lightspark.py:433,443,449,457,463) followed by the GEMV above, as
 * LiteSparkQwen._projection does it (cpu_lightspark.py:351-371).
 * Optional outputs (NULL to skip): q_out int8 [width], act_scale_out fp32
 * [1], acc_out int32 [rows] (the exact integer accumulators). */
int hq_quant_int4_gemv(const float* x, const uint8_t* weights, const float* scales,
                       float* output, int rows, int width, int8_t* q_out,
                       float* act_scale_out, int32_t* acc_out, void* stream);

/* ------------------------------------------------- quantization --
 * Per-token int8 quantization alone (kernel.quantize_activation,
 * cpu_lightspark.py:433): q int8 [n], act_scale fp32 [1] on the device. */
int hq_quantize_activation(const float* x, int n, int8_t* q, float* act_scale, void* stream);

/* ------------------------------------------------------ RMSNorm --
 * RMSNorm y = (x / sqrt(mean(x^2) + eps)) * gamma over n values
 * (kernel.rmsnorm_into, cpu_lightspark.py:431,447,461). */
int hq_rmsnorm(const float* x, const float* gamma, float* y, int n, float eps, void* stream);

/* ------------------------------------------- GQA decode attention --
 * Fused single-token GQA attention: score, softmax and V accumulation in
 * one launch (per 64-position chunk, with the chunks' combine in the same
 * launch).  Replaces litespark_gqa_decode (cpu_kernels/
 * litespark_int4.cpp:160-171, bound at cpu_lightspark.py:102-111) with the
 * same argument list and meaning:
 * query fp32 [kv_heads*groups, head_dim], heads ordered [kv_head, group];
 * keys/values fp16 (IEEE binary16 bits) [time, kv_heads, head_dim], element
 * (t, h, d) at t*kv_heads*head_dim + h*head_dim + d (the time stride is
 * derived as in litespark_int4.cpp:172); output fp32 like query.
 * score_stride is the row stride of the reference's `scores` scratch
 * [kv_heads*groups, score_stride] (the caller passes state.capacity,
 * cpu_lightspark.py:405), so context <= score_stride.  `workspace` takes the
 * place of that scratch: at least hq_gqa_workspace_bytes(score_stride, ...)
 * bytes, 256-byte aligned, zero-filled before its first use: a call hands
 * the chunk partials between its blocks through words that are nonzero once
 * written, and clears every word it used before it returns, so the
 * workspace is zero again after each call; one workspace serves every call
 * with the same or a smaller score_stride.  Calls sharing a workspace must
 * not overlap.  head_dim in {16, 32, 64, 128}; groups <= 8; context >= 1;
 * keys and values 16-byte aligned. */
size_t hq_gqa_workspace_bytes(int score_stride, int kv_heads, int groups, int head_dim);
int hq_gqa_decode(const float* query, const uint16_t* keys, const uint16_t* values,
                  void* workspace, float* output, int context, int kv_heads, int groups,
                  int head_dim, int score_stride, void* stream);

/* hq_gqa_decode without the workspace argument: the variant that allocates
 * nothing.  No counterpart in the reference; it is for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that
 * forbid hipMalloc).  Same arguments, checks and results as hq_gqa_decode;
 * the workspace is a 4 MiB file-scope device array that each GPU holds until
 * the process ends, so the call returns HQ_ERR_ARG when
 * hq_gqa_workspace_bytes(context, kv_heads, groups, head_dim) exceeds 4 MiB
 * (32 query heads of 128 dims: context <= 15872).  Every call on a GPU shares
 * that GPU's array: calls that overlap on one GPU race.  The array starts
 * zero-filled and every call leaves it zero (as hq_gqa_decode leaves its
 * workspace); no hipMalloc, hipFree or memset is called. */
int hq_gqa_decode_noalloc(const float* query, const uint16_t* keys, const uint16_t* values,
                          float* output, int context, int kv_heads, int groups, int head_dim,
                          int score_stride, void* stream);

/* ------------------------------------------------------- argmax --
 * Device argmax with np.argmax's order: the first maximal index, a NaN
 * beating every number (cpu_lightspark.py:704-705, the greedy branch of
 * sample_logits).  out_index int32 [1].  `workspace`:
 * hq_argmax_workspace_bytes(n) bytes, 256-byte aligned, zero-filled before
 * its first use; it serves any later call with no larger n. */
size_t hq_argmax_workspace_bytes(int n);
int hq_argmax(const float* x, int n, int32_t* out_index, void* workspace, void* stream);

/* --------------------------------------------- stochastic sampler --
 * Stochastic sampling of one token (the non-argmax branch of sample_logits,
 * cpu_lightspark.py:706-726): repetition penalty over the ids in
 * `generated` (repeats count once), temperature, the top_k largest values
 * (value descending, equal values by ascending index), softmax, top-p
 * (probabilities whose preceding cumulative mass reaches top_p set to 0,
 * renormalised), then numpy Generator.choice's inverse-cdf draw with the
 * uniform number *u (device double in [0,1), e.g. the host generator's
 * random()).  logits fp32 [n]; generated int32 [n_generated] (ids outside
 * [0,n) are skipped); out_token int32 [1]; ids_out int32 [k] and probs_out
 * fp32 [k] (nullable) receive the ranked ids and final probabilities, k =
 * min(top_k, n).  1 <= top_k <= 2048, temperature > 0, repetition_penalty
 * > 0, top_p > 0 (>= 1: no top-p filtering).  One launch: each block
 * radix-selects the top k of its 4096 logits, the last block to finish (a
 * ticket counter in the workspace) selects and sorts the overall top k and
 * draws.  `workspace`: hq_sample_workspace_bytes(n, top_k) bytes, 256-byte
 * aligned, zero-filled before its first use; every call leaves the counter
 * at zero, so a workspace serves later calls with any n and top_k it is
 * large enough for.  Calls sharing a workspace must not overlap. */
size_t hq_sample_workspace_bytes(int n, int top_k);
int hq_sample_token(const float* logits, int n, const int32_t* generated, int n_generated,
                    float repetition_penalty, float temperature, int top_k, float top_p,
                    const double* u, int32_t* out_token, int32_t* ids_out, float* probs_out,
                    void* workspace, void* stream);

/* -------------------------------------------------- batched GEMM --
 * Batched decode (M concurrent sequences share each weight read).  No
 * reference counterpart (forward_token is batch 1, cpu_lightspark.py:424);
 * defined as M independent hq_int4_i8_gemv calls and bit-identical to them:
 *   output[m, n] = ((float)sum_k W[n,k] * x[m,k] * act_scales[m]) * scales[n]
 * x int8 [m, width]; act_scales fp32 [m]; output fp32 [m, rows];
 * acc_out (nullable) int32 [m, rows].  The products run on int8 MFMA
 * (v_mfma_i32_16x16x64_i8); a block owns whole rows over the whole K (its
 * waves split K and add their int32 partial tiles in LDS), so no partial
 * sum crosses blocks.  `workspace` (hq_gemm_workspace_bytes(m, rows, width)
 * bytes, 16-byte aligned, zero-filled before its first use) holds the
 * activations re-laid out for the MFMA operands: m rows padded to a
 * multiple of 32, width padded to a multiple of 256 columns, even/odd
 * columns de-interleaved per 8, stored in tiles of 16 rows in the order the
 * 64 lanes of an MFMA B operand load them (each 128-column step of a tile
 * as two 1 KB blocks), then (hq_quant_int4_gemm) the m activation
 * scales.  A call never writes the padding, which must stay zero, so a
 * workspace may be reused by later calls of the same m and width; give
 * calls of other shapes their own workspace.  width % 32 == 0, weights
 * 16-byte aligned, 1 <= m. */
size_t hq_gemm_workspace_bytes(int m, int rows, int width);
int hq_int4_i8_gemm(const int8_t* x, const float* act_scales, const uint8_t* weights,
                    const float* scales, float* output, int m, int rows, int width,
                    int32_t* acc_out, void* workspace, void* stream);
/* Fused form: per-sequence quantization of fp32 x [m, width] (hq_quantize_activation's spec
 * applied to each row), then the GEMM.  q_out int8 [m, width] and
 * act_scales_out fp32 [m] are optional outputs.  Here width <= 10240, x is
 * 16-byte aligned and q_out (when given) 8-byte aligned. */
int hq_quant_int4_gemm(const float* x, const uint8_t* weights, const float* scales,
                       float* output, int m, int rows, int width, int8_t* q_out,
                       float* act_scales_out, int32_t* acc_out, void* workspace,
                       void* stream);

/* ----------------------------------------------------- decode step --
 * One decode step of a Qwen3-shaped model, as LiteSparkQwen.forward_token
 * (cpu_lightspark.py:424-468): embedding row decode, per layer RMSNorm ->
 * quant -> fused qkv GEMV -> qk-norm -> RoPE -> fp16 KV write -> GQA
 * attention -> quant -> o GEMV + residual -> RMSNorm -> quant -> fused
 * gate_up GEMV with SwiGLU -> quant -> down GEMV + residual; final RMSNorm
 * -> quant -> tied LM head GEMV -> argmax (lowest index on ties, as
 * np.argmax at cpu_lightspark.py:704-705).
 * All pointers inside the structs are device pointers except hq_model.layer,
 * a host array of `layers` entries.  The structs are plain C.
 * When hq_model.device_layer holds a device copy of that array (and the
 * shapes fit its limits), the decoder layers of a step run as one persistent
 * kernel; otherwise as five kernels per layer.  Both give the same bits.
 * HQ_MODEL_PER_LAYER_KERNELS in hq_model.flags selects the five-kernel form. */
typedef struct hq_layer {
    const uint8_t* qkv;      const float* qkv_scales;      /* [q+2kv, hidden/2], [q+2kv] */
    const uint8_t* o;        const float* o_scales;        /* [hidden, q/2], [hidden] */
    const uint8_t* gate_up;  const float* gate_up_scales;  /* [2*inter, hidden/2] */
    const uint8_t* down;     const float* down_scales;     /* [hidden, inter/2] */
    const float* input_norm; const float* post_norm;       /* [hidden] */
    const float* q_norm;     const float* k_norm;          /* [head_dim] */
} hq_layer;

typedef struct hq_model {
    int32_t layers, hidden, intermediate, heads, kv_heads, head_dim, vocab, rope_positions;
    float eps;
    int32_t flags;                  /* HQ_MODEL_* bits */
    const hq_layer* layer;          /* HOST array [layers] */
    const uint8_t* embedding;       /* [vocab, hidden/2], tied LM head */
    const float* embedding_scales;  /* [vocab] */
    const float* final_norm;        /* [hidden] */
    const float* rope_cos;          /* [rope_positions, head_dim/2] */
    const float* rope_sin;
    const hq_layer* device_layer;   /* optional DEVICE copy of layer[] */
} hq_model;

#define HQ_MODEL_PER_LAYER_KERNELS 1

typedef struct hq_state {
    int32_t capacity;     /* KV positions */
    int32_t reserved;
    uint16_t* keys;       /* fp16 [layers, capacity, kv_heads, head_dim] */
    uint16_t* values;
    int32_t* position;    /* [1] next position; advanced by each step */
    int32_t* token;       /* [1] input token; replaced by the greedy token */
    int32_t* status;      /* [1] 0, or HQ_STEP_* bits (sticky) */
    float* x;             /* [hidden] residual stream */
    float* qkv;           /* [q+2kv] raw fused projection */
    float* attended;      /* [q] */
    float* activated;     /* [inter] SwiGLU output */
    float* logits;        /* [vocab] */
    void* workspace;      /* hq_step_workspace_bytes(); zero-filled once */
} hq_state;

#define HQ_STEP_BAD_TOKEN 1
#define HQ_STEP_FULL 2
#define HQ_STEP_SYNC 4   /* a phase wait of the persistent layer kernel gave up */

size_t hq_step_workspace_bytes(const hq_model* model, int capacity);
/* Blocks of the persistent layer kernel a step of this model launches on the
 * current device (one per CU at most), or 0 when the step runs five kernels
 * per layer.  No reference counterpart (introspection). */
int hq_step_layer_blocks(const hq_model* model);
/* Enqueue one step.  Reads *state->token and *state->position on the device,
 * so the same launch sequence serves every position (graph-capturable). */
int hq_decode_step(const hq_model* model, const hq_state* state, void* stream);

/* Batched prefill: consume tokens[0..count) (device int32) at positions
 * start .. start+count-1 layer by layer for up to 128 tokens at a time (the
 * body projections as int8 MFMA GEMMs, attention batched over the tokens,
 * each query seeing its own causal context), with the arithmetic of
 * hq_decode_step, so the K/V rows written are the bits count steps would
 * write.  No logits are computed: forward the prompt's last token with
 * hq_decode_step.  Leaves *state->position = start + count.  Bad token IDs
 * set HQ_STEP_BAD_TOKEN.  `workspace`: hq_prefill_workspace_bytes(model,
 * state->capacity) bytes, 256-byte aligned, zero-filled before first use.
 * Reference counterpart: the token-by-token prompt loop of
 * cpu_lightspark.py:809-810 and inference_runtime.py:177-181. */
size_t hq_prefill_workspace_bytes(const hq_model* model, int capacity);
int hq_prefill(const hq_model* model, const hq_state* state, const int32_t* tokens, int count, int start,
               void* workspace, void* stream);

/* Batched decode: one decode step for each of `count` (1..32) independent
 * sequences, each with its own hq_state (KV cache, position, token, status,
 * residual, logits), as `count` hq_decode_step calls would run them and with
 * the same bits, but sharing every weight read: per layer the body
 * projections are int8 MFMA GEMMs over the batch, attention runs over each
 * sequence's own cache and context, and the tied LM head is one GEMM over
 * the batch followed by a per-sequence argmax that writes each greedy token
 * to *state->token and advances *state->position.  No reference
 * counterpart (forward_token is batch 1, cpu_lightspark.py:424-468; the
 * reference runtime keeps one session per request, inference_runtime.py:
 * 177-184): the contract is M forward_token steps.  `states` is a HOST array
 * of count structs; every state's capacity must be <= max_capacity, the
 * capacity the workspace was sized for: hq_decode_batch_workspace_bytes(
 * model, max_capacity) bytes, 256-byte aligned, zero-filled before first use
 * (its tickets are left at zero by every call).  Its first 4 bytes hold a
 * uint32 step counter that advances by one per call and tags the values the
 * step's launches hand to their last blocks; a launch accepts only values
 * tagged with its own step and launch.  The counter runs 1 .. 2^23 - 1: the
 * call that would pass 2^23 - 1 (or finds the counter outside that range)
 * first clears every tagged value and restarts at 1, so the workspace can
 * serve any number of calls.  A full cache sets
 * HQ_STEP_FULL and a bad token HQ_STEP_BAD_TOKEN in that state's status.
 * Shapes: those hq_prefill takes, with at most 64 query heads and a hidden
 * size of at most 4096 (the workspace size is 0 and the call HQ_ERR_ARG
 * otherwise). */
size_t hq_decode_batch_workspace_bytes(const hq_model* model, int max_capacity);
int hq_decode_batch(const hq_model* model, const hq_state* states, int count, int max_capacity,
                    void* workspace, void* stream);

/* Launch one body GEMV of the step (the kernel the step launches) for one
 * layer on the state's buffers, so a kernel can be timed in isolation.
 * kind: 0 = RMSNorm+qkv, 1 = o + residual, 2 = RMSNorm+gate_up+SwiGLU,
 * 3 = down + residual.  No reference counterpart (measurement hook). */
int hq_step_gemv(const hq_model* model, const hq_state* state, int layer, int kind,
                 void* stream);

/* Launch only the decoder layers of a step (the persistent layer kernel, or
 * the five kernels per layer) on the state's buffers, at the state's current
 * position, without the embedding, LM head or position advance, so their
 * time can be measured alone.  No reference counterpart (measurement hook). */
int hq_step_layers(const hq_model* model, const hq_state* state, void* stream);

/* Capture `steps` consecutive decode steps enqueued on `stream` (which must
 * not be the default stream) into an executable HIP graph. */
int hq_graph_capture(const hq_model* model, const hq_state* state, int steps,
                     void* stream, void** graph_exec);
int hq_graph_launch(void* graph_exec, void* stream);
int hq_graph_destroy(void* graph_exec);

#ifdef __cplusplus
}
#endif
#endif
