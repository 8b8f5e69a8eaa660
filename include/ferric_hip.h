/*
 * ferric_hip.h — C ABI of the MI355X (gfx950) Qwen3 forward-pass hot path.
 *
 * This library replaces the GPU work behind Ferric's batch-runner boundary:
 *
 *   trait EngineeringTpBatchRunnerV2::execute_batch(&EngineeringTpPreparedBatchV1,
 *                                                   output_rows) -> choices
 *   (adapters/m1-engineering-execution-v1/src/tp_batch_runtime.rs:20-95)
 *
 * as implemented by EngineeringTpBatchExecutionV2::forward
 * (adapters/m1-engineering-execution-v1/src/tp_execution/batched.rs:1746-2454).
 * The caller (scheduler + paged pool, tp_batch_runtime.rs:314-480) keeps page
 * ownership; this library owns weights and KV device memory, allocated once.
 *
 * Conventions: every function returns an fh_status; nothing throws across the
 * ABI. Host buffers are caller-owned. One HIP stream per context; calls on one
 * context must come from one thread at a time (the reference's single
 * controller thread, tp_execution.rs:92-99). bf16 values are uint16_t carriers
 * (round-to-nearest-even narrowing, NaN quieted with |0x40).
 *
 * The fh_op_* entry points run one kernel family on caller-provided device
 * pointers and a caller-provided stream (hipStream_t passed as void*). They
 * are the kernel roots of the K1-K7 catalog (crates/ferric-kernels/src/
 * catalog.rs:47-65) and are what the parity tests drive.
 */
#ifndef FERRIC_HIP_H
#define FERRIC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Errors mirror the reference's TpResult<String> failure classes
 * (tp_execution.rs:43; batched.rs:1678-1744, 1519-1530). */
typedef enum fh_status {
  FH_OK = 0,
  FH_ERR_INVALID_ARGUMENT = 1, /* bad pointer, shape or descriptor */
  FH_ERR_INVALID_BATCH = 2,    /* "foreign, stale, or invalid prepared GPU batch" */
  FH_ERR_INVALID_ROW = 3,      /* "invalid paged row geometry or aliased write slot" */
  FH_ERR_SHARED_PAGE = 4,      /* "batch writes a page shared with another sequence or logical position" */
  FH_ERR_OUTPUT_ROWS = 5,      /* "output rows must be unique, ascending, and within the batch" */
  FH_ERR_NONFINITE = 6,        /* a kernel saw a nonfinite value or an out-of-range index (reference: trap) */
  FH_ERR_DEVICE = 7,           /* HIP runtime failure */
  FH_ERR_POISONED = 8,         /* a previous batch failed; only fh_destroy recovers */
  FH_ERR_OUT_OF_MEMORY = 9,
  FH_ERR_STATE = 10            /* weights or KV pool not ready */
} fh_status;

/* Tensor kinds, in the reference's order (crates/ferric-spec/src/qwen3.rs:20-35). */
typedef enum fh_tensor_kind {
  FH_LANGUAGE_MODEL_HEAD = 0,
  FH_TOKEN_EMBEDDING = 1,
  FH_FINAL_NORM = 2,
  FH_INPUT_LAYER_NORM = 3,
  FH_POST_ATTENTION_LAYER_NORM = 4,
  FH_QUERY_NORM = 5,
  FH_KEY_NORM = 6,
  FH_QUERY_PROJECTION = 7,
  FH_KEY_PROJECTION = 8,
  FH_VALUE_PROJECTION = 9,
  FH_OUTPUT_PROJECTION = 10,
  FH_GATE_PROJECTION = 11,
  FH_UP_PROJECTION = 12,
  FH_DOWN_PROJECTION = 13
} fh_tensor_kind;

/* Model shape; mirrors the admitted Qwen3 configuration
 * (crates/ferric-spec/src/configuration.rs:107-194). head_dim must be 128,
 * kv_heads 8, hidden/intermediate multiples of 256. */
typedef struct fh_model_desc {
  uint32_t layers;         /* 36 (8B) / 28 (0.6B) */
  uint32_t hidden;         /* 4096 / 1024 */
  uint32_t query_heads;    /* 32 / 16 */
  uint32_t kv_heads;       /* 8 */
  uint32_t head_dim;       /* 128 */
  uint32_t intermediate;   /* 12288 / 3072 */
  uint32_t vocabulary;     /* 151936 */
  uint32_t tied_embedding; /* 0 (8B) / 1 (0.6B): LM head reads the embedding table */
  uint32_t rope_theta;     /* 1000000, an integer as in rope_bytes (tp_execution.rs:1440) */
  float rms_epsilon;       /* 1e-6 */
} fh_model_desc;

/* Resident-state envelope; mirrors EngineeringTpPagedLimitsV1 (tp_paged.rs:257-350). */
typedef struct fh_ctx_options {
  uint32_t row_capacity;      /* rows per batch, 1..32 (reference wide profile: 32) */
  uint32_t physical_pages;    /* KV pages per layer in the pool */
  uint32_t page_table_stride; /* page-table entries per row (context_tokens / 16, rounded up) */
  uint32_t context_tokens;    /* positions must be < context_tokens */
  uint32_t use_graphs;        /* 1: replay one HIP graph per row count */
  uint32_t capture_hidden;    /* 1: keep every layer's residual output for fh_read_hidden */
  int32_t device;             /* HIP device ordinal */
  uint32_t prefill_rows;      /* 0, or the largest batch (> row_capacity) run as a prefill chunk */
} fh_ctx_options;

/* One prepared row; mirrors EngineeringTpPreparedRowV1 (tp_paged.rs:257-300). */
typedef struct fh_row {
  uint64_t sequence;      /* opaque sequence identity */
  uint32_t token;         /* input token id (< vocabulary) */
  uint32_t position;      /* absolute position; the KV slot written is pages[position/16], position%16 */
  const uint32_t* pages;  /* logical-to-physical page list */
  uint32_t page_count;    /* <= page_table_stride */
  uint32_t writable_page; /* must equal pages[position / 16] */
} fh_row;

typedef struct fh_ctx fh_ctx;

/* ---- context lifecycle (replaces the worker/transport setup of
 *      EngineeringTpBatchExecutionV2; tp_execution.rs:99-230) ---- */

/* Creates a context: weight storage, KV pool, RoPE table, workspaces. */
fh_status fh_create(const fh_model_desc* model, const fh_ctx_options* options, fh_ctx** out);
/* Releases every device allocation (replaces close(), tp_batch_runtime.rs:93). */
void fh_destroy(fh_ctx* ctx);
/* Message of the last failure on this context, or, when ctx is NULL, of the
   last failed fh_create or fh_op_* launch on the calling thread. */
const char* fh_last_error(const fh_ctx* ctx);

/* Uploads one row-major bf16 weight [N][K] (nn.Linear layout; norms are [width]).
 * Replaces the per-rank weight upload (tp_execution.rs:272, UPLOAD_CHUNK_BYTES).
 * Projections are re-laid out on the device into MFMA tile order. */
fh_status fh_upload_weight(fh_ctx* ctx, uint32_t kind, uint32_t layer, const uint16_t* host_bf16,
                           uint64_t elements);
/* Generates every weight on the device with the ferric_synth.h convention
 * (projections/embedding ~N(0, sigma), norms = 1.0). */
fh_status fh_synthesize_weights(fh_ctx* ctx, uint64_t seed, float sigma);
/* Reads one weight back in row-major order (parity tests). */
fh_status fh_download_weight(fh_ctx* ctx, uint32_t kind, uint32_t layer, uint16_t* host_bf16,
                             uint64_t elements);

/* Fills KV positions [0, rows[i].position) of each row's sequence in every layer
 * with ferric_synth.h samples keyed by (sequence_keys[i], position, head, dim). */
fh_status fh_kv_fill_synthetic(fh_ctx* ctx, uint64_t seed, float sigma, const fh_row* rows,
                               const uint64_t* sequence_keys, uint32_t nrows, uint32_t context_stride);
/* Copies one physical KV page ([16][kv_heads][head_dim] bf16) of one layer. which: 0 = K, 1 = V. */
fh_status fh_read_kv_page(fh_ctx* ctx, uint32_t layer, uint32_t which, uint32_t page, uint16_t* out,
                          uint64_t elements);
fh_status fh_write_kv_page(fh_ctx* ctx, uint32_t layer, uint32_t which, uint32_t page,
                           const uint16_t* data, uint64_t elements);
/* Copies one layer's whole K or V pool ([physical_pages][16][kv_heads][head_dim] bf16;
 * elements must be that size): a parity readback, like fh_read_kv_page. */
fh_status fh_read_kv_cache(fh_ctx* ctx, uint32_t layer, uint32_t which, uint16_t* out, uint64_t elements);

/* ---- the hot path ---- */

/* Runs one forward step over the prepared rows and writes the greedy choice of
 * each requested output row (ascending row indices) to choices_out[nout].
 * Up to row_capacity rows run the decode path (weight-streaming projections,
 * one HIP graph per row count); larger batches, up to prefill_rows, run the
 * prefill path (compute-bound MFMA projections; logits only for output rows;
 * fh_read_logits then returns the output rows' logits in output order).
 * Replaces EngineeringTpBatchRunnerV2::execute_batch (tp_batch_runtime.rs:51-58)
 * / EngineeringTpBatchExecutionV2::forward (batched.rs:1746-2454). batch_id must
 * increase strictly (batched.rs:1700). On failure nothing is published and the
 * context is poisoned (tp_batch_runtime.rs:474). */
fh_status fh_execute_batch(fh_ctx* ctx, uint64_t batch_id, const fh_row* rows, uint32_t nrows,
                           const uint32_t* output_rows, uint32_t nout, uint32_t* choices_out);

/* Parity readbacks of the last batch: FP32 logits [nrows][vocabulary] (prefill: the
 * output rows, in output order); the residual stream after layer `layer`
 * [nrows][hidden] for every token row of the batch (needs capture_hidden, which
 * holds max(row_capacity, prefill_rows) rows per layer). */
fh_status fh_read_logits(fh_ctx* ctx, float* out, uint64_t elements);
fh_status fh_read_hidden(fh_ctx* ctx, uint32_t layer, uint16_t* out, uint64_t elements);

/* Rows the runner accepts per batch (row_capacity(), tp_batch_runtime.rs:47). */
uint32_t fh_row_capacity(const fh_ctx* ctx);
/* Kernel launches issued by successful batches (dispatch_counts(), tp_batch_runtime.rs:89). */
uint64_t fh_dispatch_count(const fh_ctx* ctx);
/* Preflight: the increment of fh_dispatch_count that fh_execute_batch with the same arguments
 * will make, evaluated without launching anything (the step's own enqueue code, run dry). The
 * batch is validated first, with fh_execute_batch's error classes. The count depends on the
 * batch: decode steps take 7, 8 or 9 launches per layer (the QK-norm/KV append runs inside the
 * attention partitions when no row reads another row's new slot and the shape allows it; the
 * partition merge runs in the same launch for small launches), prefill chunks another schedule,
 * and capture_hidden adds copies. Replaces expected_dispatch_counts_for_selection
 * (tp_batch_runtime.rs:80-86; the reference's per-batch policy is tp_execution/batched.rs:1494-1560),
 * whose result the caller compares with the dispatch_counts() increment (tp_batch_runtime.rs:432-446). */
fh_status fh_expected_dispatch_count(fh_ctx* ctx, uint64_t batch_id, const fh_row* rows, uint32_t nrows,
                                     const uint32_t* output_rows, uint32_t nout, uint64_t* count);
/* Device milliseconds of the last fh_execute_batch, from HIP events on the context stream. */
float fh_last_step_ms(const fh_ctx* ctx);
/* Per-kernel-class device time of the last batch when profiling is on (parity/bench aid).
 * kernel_class indexes fh_kernel_class; returns total ms across launches of that class. */
fh_status fh_set_profiling(fh_ctx* ctx, uint32_t enabled);
fh_status fh_kernel_class_ms(const fh_ctx* ctx, uint32_t kernel_class, float* ms, uint32_t* launches);
/* Measurement aid with no counterpart in the reference: re-launches the last decode
 * batch's attention partition kernel for the last layer (same inputs, so it rewrites the
 * same outputs) reps times back to back on the context stream between two events and
 * writes the mean launch duration in ms (1 <= reps <= 1000). FH_ERR_STATE if the last
 * batch was not a decode batch. */
fh_status fh_time_attention(fh_ctx* ctx, uint32_t reps, float* avg_ms);

typedef enum fh_kernel_class {
  FH_KC_EMBEDDING = 0,
  FH_KC_RMSNORM = 1,
  FH_KC_QKV_GEMM = 2,
  FH_KC_QKNORM_ROPE_KV = 3,
  FH_KC_ATTENTION = 4,
  FH_KC_ATTENTION_MERGE = 5,
  FH_KC_O_GEMM = 6,
  FH_KC_GATE_UP_GEMM = 7,
  FH_KC_DOWN_GEMM = 8,
  FH_KC_HEAD_GEMM = 9,
  FH_KC_ARGMAX = 10,
  FH_KC_COUNT = 11
} fh_kernel_class;

/* ---- kernel roots on device pointers (K1-K7) ---- */

/* Re-lays a row-major bf16 weight [n][k] into MFMA tile order (n % 16 == 0, k % 32 == 0). */
fh_status fh_op_tile_weight(const uint16_t* src, uint16_t* dst, uint32_t n, uint32_t k, void* stream);
/* Interleaves gate [i][k] and up [i][k] into one tiled operand for the fused SwiGLU epilogue. */
fh_status fh_op_tile_gate_up(const uint16_t* gate, const uint16_t* up, uint16_t* dst, uint32_t i,
                             uint32_t k, void* stream);
/* Row-major gather back out of tile order (embedding rows; weight readback). */
fh_status fh_op_untile_weight(const uint16_t* tiled, uint16_t* dst, uint32_t n, uint32_t k, void* stream);

/* K1 embedding: out[r][:] = table[tokens[r]][:] (bit copy); table is tiled [vocab][hidden].
 * Replaces ferric_qwen3_token_embedding_bf16_copy_v1 (device/qwen3-all-kernels-v1/src/gemm.rs:768). */
fh_status fh_op_embedding(const uint32_t* tokens, const uint16_t* table_tiled, uint16_t* out,
                          uint32_t rows, uint32_t hidden, uint32_t vocabulary, uint32_t* error_word,
                          void* stream);

/* K2 RMSNorm over width 1024/4096 (pure mode) with a wavefront reduction.
 * Replaces qwen3_rmsnorm_v1 behavior 0 (rmsnorm.rs:380) / wave_rmsnorm_bf16_v15. */
fh_status fh_op_rmsnorm(const uint16_t* x, const uint16_t* weight, uint16_t* y, uint32_t rows,
                        uint32_t width, float epsilon, uint32_t* error_word, void* stream);

/* K1 projections: out = epilogue(x[m][k] . W[n][k]^T) with FP32 accumulation on MFMA.
 * epilogue: FH_EPI_BF16 (one RNE), FH_EPI_RESIDUAL (bf16((0 + acc) + residual), may alias out),
 * FH_EPI_SWIGLU (w from fh_op_tile_gate_up, n = 2*i, out [m][i] = swiglu(bf16(g), bf16(u))),
 * FH_EPI_F32 (FP32 out, the LM head). m <= 32 streams the weight (decode, split-K allowed);
 * m > 32 needs n % 128 == 0 and ldo % 4 == 0: up to 256 rows FH_EPI_PARTIAL, FH_EPI_SWIGLU
 * and FH_EPI_F32 run the panel kernel (activation panel shared through LDS; split-K allowed
 * for FH_EPI_PARTIAL), the other epilogues the weight-streaming kernel over row chunks
 * (splits = 1); beyond 256 rows the compute-bound prefill kernel (256 x 256 blocks through
 * LDS when n % 256 == 0, else 128 x 128 blocks; splits = 1, no FH_EPI_PARTIAL). Replaces
 * gemm.rs:161/:605 and
 * device/qwen3-tp-batch32-kernels-v5/src/projection.rs:15/:142/:241, collective.rs:25,
 * activation.rs:32 and device/qwen3-tp-fp32-head32-kernels-v8/src/projection.rs:66/:186. */
enum { FH_EPI_BF16 = 0, FH_EPI_RESIDUAL = 1, FH_EPI_SWIGLU = 2, FH_EPI_F32 = 3, FH_EPI_PARTIAL = 4 };
/* x_tiled is in activation tile order (fh_op_tile_activation). FH_EPI_SWIGLU writes its
 * output in activation tile order (the down projection's input); FH_EPI_PARTIAL writes
 * FP32 partial sums as `splits` slabs of [fh_partial_slab_rows(m)][ldo] (split-K across
 * workgroups; the consumer adds the slabs in order and rounds once; a split past the end
 * of k writes zeros). Other epilogues use splits = 1.
 * error_word (may be NULL) receives the nonfinite bit where the SwiGLU epilogue meets a
 * nonfinite gate, up or product (qwen3_swiglu_bf16_f32_v1 traps there). */
fh_status fh_op_gemm(const uint16_t* x_tiled, const uint16_t* w_tiled, uint32_t m, uint32_t n, uint32_t k,
                     uint32_t epilogue, uint32_t splits, const uint16_t* residual, void* out, uint32_t ldo,
                     uint32_t* error_word, void* stream);
/* Split-K factor the runtime uses for an n x k projection. */
uint32_t fh_gemm_default_splits(uint32_t n, uint32_t k);
/* Rows a tiled activation buffer for m rows holds: 32 for m <= 32, else m rounded up to 256. */
uint32_t fh_activation_rows(uint32_t m);
/* Rows of one FH_EPI_PARTIAL slab for an m-row batch: 32 for m <= 32, 256 for 32 < m <= 256,
 * 0 (no split-K partials) otherwise. No counterpart in the reference, whose split-K
 * partials are per-step buffers of its decode path (v5 collective.rs:25-60). */
uint32_t fh_partial_slab_rows(uint32_t m);
/* Row-major [m][k] bf16 <-> activation tile order (the tiled buffer holds fh_activation_rows(m) x k). */
fh_status fh_op_tile_activation(const uint16_t* x, uint16_t* x_tiled, uint32_t m, uint32_t k, void* stream);
fh_status fh_op_untile_activation(const uint16_t* x_tiled, uint16_t* x, uint32_t m, uint32_t k, void* stream);

/* K2 residual + RMSNorm, fused: when splits > 0, hidden[r] = bf16((0 + sum_s partials[s][r]) +
 * hidden[r]) is written back first (the TP1 residual, v5 collective.rs:25-60, with the split-K
 * slabs summed in order), then y = RMSNorm(hidden) is written in activation tile order
 * (y_tiled = 1, fh_activation_rows(rows) rows) or row-major. partials: `splits` slabs of
 * [fh_partial_slab_rows(rows)][width] FP32 (rows <= 256 when splits > 0). */
fh_status fh_op_residual_rmsnorm(uint16_t* hidden, const float* partials, uint32_t splits, const uint16_t* weight,
                                 uint16_t* y, uint32_t y_tiled, uint32_t rows, uint32_t width, float epsilon,
                                 uint32_t* error_word, void* stream);

/* K2 + K1 for one decode row: the residual + RMSNorm above (rows = 1, width = k) run by
 * every workgroup of the projection that consumes the normalized row, so the row never
 * goes through memory between them. When norm_splits > 0, hidden_out = bf16((0 + sum_s
 * partials[s][0]) + hidden_in) is written (hidden_out must not alias hidden_in); then
 * out = epilogue(RMSNorm(hidden) . W^T) as fh_op_gemm with m = 1. Bit-identical to
 * fh_op_residual_rmsnorm followed by fh_op_gemm on the same inputs. Covered: the
 * projections that follow a norm in a Qwen3 layer (FH_EPI_PARTIAL with the splits
 * fh_gemm_default_splits gives, norm_splits 0, 4 or 6; FH_EPI_SWIGLU and FH_EPI_F32 with
 * norm_splits 4 or 6), k = 1024..4096 with k % 256 == 0; FH_ERR_INVALID_ARGUMENT
 * otherwise. Fuses the two launches the reference makes per norm
 * (qwen3_rmsnorm_v1 then the projection, batched.rs:1494-1560). */
fh_status fh_op_gemm_rmsnorm(const uint16_t* hidden_in, uint16_t* hidden_out, const float* partials,
                             uint32_t norm_splits, const uint16_t* norm_weight, float epsilon,
                             const uint16_t* w_tiled, uint32_t n, uint32_t k, uint32_t epilogue, uint32_t splits,
                             void* out, uint32_t ldo, uint32_t* error_word, void* stream);
/* 1 when fh_op_gemm_rmsnorm covers this projection, else 0 (no GPU call). */
uint32_t fh_gemm_rmsnorm_supported(uint32_t n, uint32_t k, uint32_t epilogue, uint32_t splits, uint32_t norm_splits);

/* K3 per-head QK-norm + split-half RoPE + paged KV append, one launch.
 * qkv: [rows][(qh + 2*kvh) * 128] bf16 projection output when qkv_splits == 0, else
 * qkv_splits FP32 partial slabs of [fh_partial_slab_rows(rows)][(qh + 2*kvh) * 128] (rows <= 256;
 * each value = bf16 of the ordered slab sum); q_out: [rows][qh*128] rotated queries;
 * k_cache/v_cache: [pages][16][kvh][128]; cos/sin: [context][64] f32 table;
 * page_table: [rows][stride]. Replaces qwen3_rmsnorm_v1 at width 128 (batched.rs:1956-1982),
 * qwen3_rope_v1 (rope_kv.rs:102) and qwen3_paged_kv_write_v1 (rope_kv.rs:261). */
fh_status fh_op_qknorm_rope_kv(const void* qkv, uint32_t qkv_splits, const uint16_t* q_norm, const uint16_t* k_norm,
                               const float* cos_table, const float* sin_table, const uint32_t* positions,
                               const uint32_t* page_table, uint16_t* q_out, uint16_t* k_cache,
                               uint16_t* v_cache, uint32_t rows, uint32_t query_heads, uint32_t kv_heads,
                               uint32_t stride, uint32_t physical_pages, uint32_t context_tokens,
                               float epsilon, uint32_t* error_word, void* stream);

/* K4 paged GQA decode attention: split-context partitions then an ordered merge.
 * q: [rows][qh*128]; out: [rows][qh*128] bf16 row-major, or activation tile order when
 * out_tiled (the output projection's input, fh_activation_rows(rows) rows);
 * scratch: fh_attention_scratch_bytes().
 * Replaces qwen3_paged_gqa_decode_bf16_f32_v1 (paged_decode.rs:222) and the split8
 * partial/merge pair (device/qwen3-tp-c1-split8-attention-kernels-v21/src/attention.rs:16, :214). */
uint64_t fh_attention_scratch_bytes(uint32_t rows, uint32_t query_heads, uint32_t context_tokens);
fh_status fh_op_paged_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                const uint32_t* positions, const uint32_t* page_table, uint16_t* out,
                                uint32_t out_tiled, void* scratch, uint32_t rows, uint32_t query_heads,
                                uint32_t kv_heads,
                                uint32_t stride, uint32_t physical_pages, uint32_t context_tokens,
                                uint32_t* error_word, void* stream);

/* K3 + K4 in one launch pair: the QK-norm + RoPE + paged KV append of fh_op_qknorm_rope_kv
 * (same arithmetic, bit for bit) run by the attention partitions of fh_op_paged_attention.
 * qkv_partials: qkv_splits FP32 split-K slabs of [fh_partial_slab_rows(rows)][(qh + 2*kvh) * 128]
 * (rows <= 32); each partition forms its query heads from them, and the partition holding a
 * row's position appends that row's K/V to the caches and uses them. The caller must not list a
 * row's written page in another row's table (rows of one sequence in one batch read each
 * other's new slots: run fh_op_qknorm_rope_kv then fh_op_paged_attention for those).
 * Shapes: query_heads / kv_heads in {1, 2, 4}, qkv_splits == 2. out, out_tiled and scratch as
 * in fh_op_paged_attention. Replaces the same reference kernels as the two calls it fuses
 * (batched.rs:1956-1982, rope_kv.rs:102, rope_kv.rs:261, paged_decode.rs:222). */
fh_status fh_op_qknorm_paged_attention(const float* qkv_partials, uint32_t qkv_splits, const uint16_t* q_norm,
                                       const uint16_t* k_norm, const float* cos_table, const float* sin_table,
                                       const uint32_t* positions, const uint32_t* page_table, uint16_t* k_cache,
                                       uint16_t* v_cache, uint16_t* out, uint32_t out_tiled, void* scratch,
                                       uint32_t rows, uint32_t query_heads, uint32_t kv_heads, uint32_t stride,
                                       uint32_t physical_pages, uint32_t context_tokens, float epsilon,
                                       uint32_t* error_word, void* stream);

/* No counterpart in the reference: fh_op_paged_attention without a workspace, for
 * callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). The partition records live in a
 * static device array of the library: 16384 records = 8.5 MB, held on every GPU the
 * library has launched on until the process ends. A launch needs rows x query_heads x
 * ceil(context_tokens / (16 x split_pages)) records, where split_pages is 32 (512-token
 * partitions) when 256 < context_tokens <= 512, else 16 (256-token partitions) when
 * rows x query_heads <= 64 or query_heads <= 16, else 32; larger launches return
 * FH_ERR_INVALID_ARGUMENT.
 * Calls that overlap on one GPU share that array and race. Same kernels and results
 * as fh_op_paged_attention. */
fh_status fh_op_paged_attention_noalloc(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                        const uint32_t* positions, const uint32_t* page_table, uint16_t* out,
                                        uint32_t out_tiled, uint32_t rows, uint32_t query_heads, uint32_t kv_heads,
                                        uint32_t stride, uint32_t physical_pages, uint32_t context_tokens,
                                        uint32_t* error_word, void* stream);

/* K6 SwiGLU as its own kernel: out = bf16(silu(g) * u), the stable-sigmoid form of
 * qwen3_swiglu_bf16_f32_v1 (device/qwen3-all-kernels-v1/src/swiglu.rs:62-120). */
fh_status fh_op_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, uint64_t elements,
                       uint32_t* error_word, void* stream);

/* K7 two-pass lowest-id argmax over FP32 logits [rows][vocabulary]; scratch:
 * fh_argmax_scratch_bytes(). Replaces device/qwen3-tp-fp32-sharded-argmax-kernels-v13/src/
 * logits.rs:87/:178 (and the serial v8 logits.rs:30 semantics). */
uint64_t fh_argmax_scratch_bytes(uint32_t rows);
fh_status fh_op_argmax(const float* logits, uint32_t rows, uint32_t vocabulary, void* scratch,
                       uint32_t* choices, uint32_t* error_word, void* stream);

/* Fills dst[0..count) with ferric_synth.h samples of (tensor_seed, index), scale from fh_synth_scale(). */
fh_status fh_op_synth_fill(uint16_t* dst, uint64_t count, uint64_t tensor_seed, float scale, void* stream);

/* Speculative decoding helpers (integer work), mirrors of
 * ferric_qwen3_speculative_token_assembly_v1 (logits.rs:587) and
 * verify_greedy_round (crates/ferric-spec/src/speculation.rs:126). */
/* target_ids[s][0] = anchors[s]; target_ids[s][1 + i] = draft[i][s] (draft is iteration-major [k][s]). */
fh_status fh_speculative_token_assembly(const uint32_t* anchors, const uint32_t* draft, uint32_t sequences,
                                        uint32_t k, uint32_t* target_ids);
/* accepted = longest prefix with draft[i] == target[i]; emitted = draft[0..accepted] + target[accepted].
 * Returns FH_ERR_INVALID_ARGUMENT unless target_count == draft_count + 1. */
fh_status fh_verify_greedy_round(const uint32_t* draft, uint32_t draft_count, const uint32_t* target,
                                 uint32_t target_count, uint32_t* accepted, uint32_t* emitted,
                                 uint32_t* emitted_count);
/* fh_verify_greedy_round for every sequence of a round in one call: draft is iteration-major
 * [k][sequences] (as fh_speculative_token_assembly takes it), target is [sequences][k + 1] (the
 * verify batch's choices); accepted[s] and emitted[s][0 .. accepted[s]] as for one sequence.
 * No counterpart in the reference, which settles sequence by sequence (speculation.rs:126);
 * for callers that settle a whole round at once. */
fh_status fh_verify_greedy_batch(const uint32_t* draft, const uint32_t* target, uint32_t sequences, uint32_t k,
                                 uint32_t* accepted, uint32_t* emitted);

/* Per-sequence 120-byte completion records [sequences][120] of
 * ferric_qwen3_compact_completion_v1 (device/qwen3-all-kernels-v1/src/logits.rs:279):
 * slot u32 | generation u32 | epoch u64 | plan identity [32] | accepted u8 |
 * emitted u8 | 0 0 | emitted tokens u32[17] (draft prefix, then the correction or
 * bonus token; zeros after). choices: [sequences][active_tokens] (sequence-major);
 * draft: [speculative_k][sequences] (iteration-major; NULL when speculative_k = 0,
 * the direct profile, which emits the choice of the last live row). A sequence
 * with active_lengths[s] = 0 gets an all-zero record. Returns
 * FH_ERR_INVALID_ARGUMENT, writing nothing, where the reference kernel traps
 * (live length, slot >= 32, generation 0, all-zero plan, a compared or emitted
 * token >= 151936) or for bad geometry (1..32 sequences; speculative_k <= 16 with
 * active_tokens = speculative_k + 1). Host-only: no device work. */
fh_status fh_compact_completion(const uint32_t* choices, const uint32_t* draft, const uint32_t* active_lengths,
                                const uint32_t* request_slots, const uint32_t* request_generations,
                                const uint64_t* completion_epochs, const uint8_t* plan_identities, uint32_t sequences,
                                uint32_t active_tokens, uint32_t speculative_k, uint8_t* records);

#ifdef __cplusplus
}
#endif

#endif /* FERRIC_HIP_H */
