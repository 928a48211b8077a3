// hq_internal.h - launch interfaces shared by the translation units of libhq.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hq.h"

namespace hq {

// ---- GEMV ------------------------------------------------------------------
enum Prologue { PRO_I8 = 0, PRO_QUANT = 1, PRO_RMSNORM = 2 };
enum Epilogue { EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_SWIGLU = 2, EPI_ARGMAX = 3 };

struct GemvParams {
    const uint8_t* w;       // [rows, width/2] packed int4
    const float* ws;        // [rows] row scales
    int rows;               // output rows (EPI_SWIGLU: 2 * half_rows)
    int width;              // K
    const float* xf;        // fp32 activations (PRO_QUANT, PRO_RMSNORM)
    const int8_t* xq;       // int8 activations (PRO_I8)
    float act_scale;        // PRO_I8 multiplier
    const float* gamma;     // PRO_RMSNORM weight [width]
    float eps;
    float* out;             // STORE/ARGMAX: [rows]; RESIDUAL: x += ; SWIGLU: [half_rows]
    float* out_aux;         // nullable: RESIDUAL projection [rows]; SWIGLU gate|up [rows]
    int32_t* acc_out;       // nullable: int32 accumulators [rows]
    int8_t* q_out;          // nullable: quantized activations [width] (block 0)
    float* act_out;         // nullable: act scale [1] (block 0)
    int half_rows;          // EPI_SWIGLU
    float* part_val;        // EPI_ARGMAX partials [blocks]
    int32_t* part_idx;
    int32_t* counter;       // EPI_ARGMAX arrival counter (zero between launches)
    int32_t* token;         // EPI_ARGMAX result
    int32_t* position;      // EPI_ARGMAX: advanced by one
};

enum class StepGemv { Qkv, OResidual, GateUpSwiglu, DownResidual, LmHead };

// Number of blocks a step GEMV launches (sizes the argmax partials).
int step_gemv_blocks(StepGemv kind, int rows, int half_rows, int width);
hipError_t launch_step_gemv(StepGemv kind, const GemvParams& p, hipStream_t s);

// ---- attention ---------------------------------------------------------------
constexpr int kAttnChunk = 64;   // positions per split (the spec's chunk)

// Per-sequence device pointers of a batched decode step (hq_decode_batch):
// sequence z has its own KV cache, position, token, status, residual and
// logits.  Lives in the step's workspace (written by a kernel from a launch
// argument, so a captured graph replays it).
constexpr int kMaxDecodeBatch = 32;
struct BatchTable {
    uint16_t* keys[kMaxDecodeBatch];     // fp16 [layers, capacity, kv_heads, head_dim]
    uint16_t* values[kMaxDecodeBatch];
    int32_t* position[kMaxDecodeBatch];
    int32_t* token[kMaxDecodeBatch];
    int32_t* status[kMaxDecodeBatch];
    float* x[kMaxDecodeBatch];
    float* logits[kMaxDecodeBatch];
    int32_t capacity[kMaxDecodeBatch];
    int32_t count;
};

struct AttnParams {
    // PLAIN mode: q given; STEP mode: raw qkv + norms + rope + KV write
    const float* q;             // PLAIN: [kv*groups, D]
    const float* qkv;           // STEP: [(heads + 2*kv) * D]
    const float* q_norm;        // STEP
    const float* k_norm;        // STEP
    const float* rope_cos;      // STEP [positions, D/2]
    const float* rope_sin;
    float eps;
    uint16_t* keys;             // fp16 cache base of this layer
    uint16_t* values;
    long long time_stride;      // elements between consecutive positions
    const int32_t* position;    // STEP: device position (context = pos + 1)
    int32_t capacity;           // STEP: bound for the KV write
    int32_t* status;            // STEP: error flag
    int context;                // PLAIN: positions of query 0
    int batch;                  // PLAIN: queries (grid z); query z sees context + z positions,
                                // reads q + z*heads*D, writes out + z*heads*D and uses its own
                                // part region (max_chunks apart)
    int kv_heads, groups, head_dim;
    int max_chunks;             // grid.y
    float* part;                // [heads, max_chunks, head_dim + 2]
    float* out;                 // [heads, D]
    // PLAIN batches of a batched decode step (nullable): query z attends the
    // cache of sequence z (layer `layer`) up to its position, table->position[z]
    // + 1 positions; keys, values and context above are then unused.  With
    // qkv set as well, query z is computed from row z of the raw projection
    // as in STEP mode (the current k/v go to sequence z's cache), and
    // launch_batch_attention quantizes each output row into q8 (row stride
    // kp, de-interleaved) with its scale in act[z].
    const BatchTable* table;
    int layer;
    int8_t* q8;
    float* act;
    int kp;
    int cpb;                    // chunks per attention block (set by launch_batch_attention)
    // Batched-step tails (nullable): the chunk partials and single-split
    // outputs go out as {value, epoch} entries (epoch = *epoch_ctr << 8 |
    // epoch_id) and the launch's last 8 * batch blocks combine and quantize
    // the rows, an eighth of the heads each, in place of the combine kernel.
    uint64_t* ll_part;          // [batch, heads, max_chunks, D + 2]
    uint64_t* ll_out;           // [batch, heads * D]
    uint64_t* ll_max;           // [batch, 8] the parts' maxima
    const uint32_t* epoch_ctr;
    int epoch_id;
    // with the qkv GEMM in the same launch (launch_batch_qkv_attention): the
    // raw projection rows as {value, epoch} entries [batch, qkv rows]
    uint64_t* qkv_ll;
};

size_t attention_workspace_floats(int heads, int max_chunks, int head_dim);
// The batched step's qkv GEMM (x: the de-interleaved input rows, act their
// scales; w, ws: the qkv matrix, k = hidden) and attention in one launch,
// with the attention's tails (a.ll_part ...) and the raw projection as
// entries in a.qkv_ll, for up to 16 sequences (batches that take the
// per-(sequence, kv head) attention excepted).  Returns
// hipErrorNotSupported, having launched nothing, when the shapes do not
// allow it (the caller then runs gemm_run and launch_batch_attention).
hipError_t launch_batch_qkv_attention(const int8_t* x, const float* act, const uint8_t* w, const float* ws, int k,
                                      const AttnParams& a, hipStream_t s);
hipError_t launch_batch_attention(const AttnParams& a, hipStream_t s);

// ---- batched GEMM driver (hq_gemm.hip) ---------------------------------------
// x: int8 activations de-interleaved per 8 columns (even columns, then odd),
// gemm_padded_m(m) rows of gemm_padded_k(k) bytes (padding zero); act fp32
// [m]; out fp32 [m, n] = ((float)acc * act) * ws.  scratch: gemm_scratch_bytes
// (m, n, k), zero before first use (left zero by every call).
int gemm_padded_k(int k);
int gemm_padded_m(int m);
size_t gemm_scratch_bytes(int m, int n, int k);
// gate_up (w: gate rows [0, n), up rows [n, 2n)) with SwiGLU in the GEMM
// epilogue into act_out [m, n], then its quantization for the down GEMM into
// q [m, kq] (de-interleaved) and act_q [m], as the SwiGLU row kernel makes
// them.  pmax: gemm_swiglu_blocks(n) * m floats.
hipError_t gemm_run_swiglu(const int8_t* x, const float* act, const uint8_t* w, const float* ws, float* act_out,
                           int m, int n, int k, float* pmax, int8_t* q, int kq, float* act_q, hipStream_t s);
int gemm_swiglu_blocks(int n);

// The batched step's o and down GEMMs with the next GEMM's input rows in
// their tail: the outputs go to ll as {value, epoch} entries and the last m
// blocks each finish one sequence's row (residual add into x, RMSNorm with
// gamma, quantization into q / act), as the RESID_NORM row kernel does.
struct GemmTail {
    uint64_t* ll;               // [m, n]
    const uint32_t* epoch_ctr;  // the step counter (advanced, and wrapped, by the step's first kernel)
    int epoch_id;               // 0 .. 255, unique per launch within a step
    float* x;                   // [m, n] residual rows, updated
    const float* gamma;         // [n]
    float eps;
    int8_t* q;                  // [m, kq] de-interleaved, zero past n
    int kq;
    float* act;                 // [m]
    const BatchTable* table;    // status words of the sequences
    uint64_t* pmax;             // gate_up: [blocks, m] entries, each block's maximum |SwiGLU| per row
};
bool gemm_tail_fits(int m, int n, int k);
bool gemm_swiglu_tail_fits(int m, int n, int k);
hipError_t gemm_run_swiglu_tail(const int8_t* x, const float* act, const uint8_t* w, const float* ws, int m, int n,
                                int k, const GemmTail& tail, hipStream_t s);
hipError_t gemm_run_tail(const int8_t* x, const float* act, const uint8_t* w, const float* ws, int m, int n, int k,
                         const GemmTail& tail, hipStream_t s);
hipError_t gemm_run(const int8_t* x, const float* act, const uint8_t* w, const float* ws, float* out, int m, int n,
                    int k, char* scratch, hipStream_t s);
hipError_t launch_attention(const AttnParams& a, bool step_mode, hipStream_t s);

// ---- persistent layer kernel ---------------------------------------------------
// Shapes the kernel is compiled for (head_dim 128, <= 4 query heads per kv
// head, hidden <= 2560, ...).
bool engine_fits(const hq_model* m);
// Grid size on the current device (0: the kernel cannot run there).
int engine_blocks(const hq_model* m);
// Bytes of hand-off words the kernel needs in the workspace (zero-filled
// before the first launch): two sets of one slot per layer.
size_t engine_handoff_bytes(const hq_model* m);
// embed: layer 0's input is the embedding row of *st->token (the step's
// lookup folded into the launch) instead of st->x.
hipError_t launch_engine(const hq_model* m, const hq_state* st, uint32_t* hs, uint32_t* epoch,
                         uint64_t* part, int max_chunks, int nb, uint32_t* trace, bool embed, hipStream_t s);
// HQ_ENGINE_TRACE builds: bytes of phase timestamps kept after the step
// workspace proper (0 otherwise).
size_t engine_trace_bytes(const hq_model* m);

}  // namespace hq
