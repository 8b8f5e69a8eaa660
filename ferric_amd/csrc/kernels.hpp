// Host-side launchers for the gfx950 kernels. Each returns the HIP error of
// the launch; shapes are validated by the callers (ops.hip / runtime.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qk_head.hpp"

namespace fh {

// Records the message fh_last_error(NULL) returns on this thread.
void set_thread_error(const char* msg);

// Attention partitions: each partition workgroup covers split_pages pages of
// 16 tokens (16 or 32; its 8 waves take split_pages / 8 pages each). Batches
// of at most 64 (row, query head) pairs, and models of at most 16 query heads
// (2 per KV head in Qwen3-0.6B, half the work per page of the 8B's 4), take
// 16-page partitions. Measured on MI355X: one Qwen3-8B row at a 4096-token
// context 13.1 us against 15.7 us for 32 pages (15.2 us for 8); 4 and 32
// rows of the 8B: 32 pages best (32 rows, contexts U[512, 8192]: attention
// 3.63 against 4.29 ms per step with 16); 32 rows of the 0.6B, contexts
// U[128, 2048]: 0.866 against 0.933 ms per step with 32 (2.04 against 2.12
// ms per step). A context capacity of 257..512 tokens takes one 32-page
// partition whatever the batch, so every row finishes in its partition with
// no records and no merge (a speculative round's 0.6B draft, 32 rows at
// 256-410 tokens of a 512-token capacity: 14.4 -> 11.8 us per launch, 1.155
// -> 1.112 ms device time per step). attn_split_pages is the one policy
// every launcher and workspace size uses.
constexpr uint32_t kAttnMaxSplitPages = 32;
constexpr uint32_t kAttnMinSplitPages = 16;
inline uint32_t attn_split_pages(uint32_t rows, uint32_t query_heads, uint32_t context_tokens) {
  if (context_tokens > kAttnMinSplitPages * 16 && context_tokens <= kAttnMaxSplitPages * 16) return kAttnMaxSplitPages;
  return (uint64_t)rows * query_heads <= 64 || query_heads <= 16 ? 16u : 32u;
}
// Floats per attention partial record: running max, denominator, numerator[128].
constexpr uint32_t kAttnPartialFloats = 2 + 128;
// Argmax first-pass shards per row.
constexpr uint32_t kArgmaxShards = 64;
// Token rows of one decode step (the activation tile order holds 2 m-tiles);
// split-K partial slabs are [kMaxRows][n] FP32.
constexpr uint32_t kMaxRows = 32;
// Prefill / wide batches (m > kMaxRows rows) run the large GEMM, whose
// workgroups cover 256 activation rows; their activation buffers hold
// act_mtiles(m) 16-row tiles (decode buffers: 2).
constexpr uint32_t kLargeBlockRows = 256;
__host__ __device__ inline uint32_t act_mtiles(uint32_t m) {
  return m <= kMaxRows ? 2u : ((m + kLargeBlockRows - 1) / kLargeBlockRows) * (kLargeBlockRows / 16);
}
// Batches of kMaxRows < m <= kPanelRows rows (a speculative verify) run the
// panel GEMM over slices of kPanelCols weight rows, which also writes split-K
// partials. A split-K partial slab holds partial_slab_rows(m) rows: 32 for
// decode batches, 256 for these.
constexpr uint32_t kPanelRows = 256;
constexpr uint32_t kPanelCols = 128;
__host__ __device__ inline uint32_t partial_slab_rows(uint32_t m) { return m <= kMaxRows ? kMaxRows : kPanelRows; }
// Whether FH_EPI_PARTIAL is supported at m rows and n output columns.
inline bool gemm_partial_rows_ok(uint32_t m, uint32_t n) {
  return m <= kMaxRows || (m <= kPanelRows && n % kPanelCols == 0);
}

inline uint32_t attn_max_splits(uint32_t context_tokens, uint32_t split_pages) {
  return (context_tokens + split_pages * 16 - 1) / (split_pages * 16);
}
// Whether a decode launch merges its partitions in the partition kernel
// (arrival counters) rather than in a second launch. Publishing the records
// coherently adds a store and counter round trip to every partition
// workgroup's life, which pays where the launch is small and costs where it
// is large. Measured on MI355X (alternating runs on one GPU, graph replays):
// one Qwen3-8B row at a 4096-token context 3.555 against 3.635 ms per step
// (16-page fused against 32-page separate merge); 32 rows of Qwen3-0.6B at
// contexts U[128, 2048] (1280 partition workgroups) 2.136 against 2.122 ms;
// 32 rows of Qwen3-8B at U[512, 8192] 12 us slower per launch fused.
inline bool attn_fuse_merge(uint32_t rows, uint32_t kv_heads, uint32_t context_tokens, uint32_t split_pages) {
  return (uint64_t)rows * kv_heads * attn_max_splits(context_tokens, split_pages) <= 1024;
}

// layout / data movement
hipError_t launch_tile_weight(const uint16_t* src, uint16_t* dst, uint32_t n, uint32_t k, uint32_t tile_mul,
                              uint32_t tile_add, hipStream_t s);
hipError_t launch_untile_weight(const uint16_t* tiled, uint16_t* dst, uint32_t n, uint32_t k, hipStream_t s);
hipError_t launch_embedding(const uint32_t* tokens, const uint16_t* table_tiled, uint16_t* out, uint32_t rows,
                            uint32_t hidden, uint32_t vocab, uint32_t* err, hipStream_t s);
hipError_t launch_synth_fill(uint16_t* dst, uint64_t count, uint64_t tensor_seed, float scale, hipStream_t s);
hipError_t launch_fill_u16(uint16_t* dst, uint64_t count, uint16_t value, hipStream_t s);
hipError_t launch_kv_fill(uint16_t* cache, const uint32_t* table, const uint32_t* lengths, const uint64_t* keys,
                          uint32_t rows, uint32_t stride, uint32_t kv_heads, uint64_t tensor_seed, float scale,
                          uint32_t context_stride, uint32_t max_length, hipStream_t s);
// dst[i] = src[index[i]] for i < rows; rows of `width` bf16 (width % 8 == 0).
hipError_t launch_gather_rows(const uint16_t* src, const uint32_t* index, uint16_t* dst, uint32_t rows,
                              uint32_t width, hipStream_t s);
hipError_t launch_clear_word(uint32_t* word, hipStream_t s);
// The first launch of a decode step (one workgroup per row): copies `words`
// 32-bit words of step metadata from coherent pinned host memory to device
// memory (in place of a host-to-device copy), sets the error word to 0 or
// ERR_TOKEN, and writes each row's embedding ([rows][hidden] row-major) for
// the token at host[row] (the block starts with the rows' tokens).
hipError_t launch_step_embed(const uint32_t* host, uint32_t* dev, uint32_t words, const uint16_t* table_tiled,
                             uint16_t* out, uint32_t rows, uint32_t hidden, uint32_t vocab, uint32_t* err,
                             hipStream_t s);
hipError_t launch_copy_u16(const uint16_t* src, uint16_t* dst, uint64_t count, hipStream_t s);

// norms / activation
hipError_t launch_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* y, uint32_t rows, uint32_t width,
                          float eps, uint32_t* err, hipStream_t s);
hipError_t launch_qknorm_rope_kv(const uint16_t* qkv, const float* qkv_part, uint32_t splits, const uint16_t* q_norm,
                                 const uint16_t* k_norm, const float* cos_t, const float* sin_t,
                                 const uint32_t* positions, const uint32_t* table, uint16_t* q_out,
                                 uint16_t* k_cache, uint16_t* v_cache, uint32_t rows, uint32_t qh, uint32_t kvh,
                                 uint32_t stride, uint32_t pages, uint32_t context, float eps, uint32_t* err,
                                 hipStream_t s);
hipError_t launch_residual_rmsnorm(uint16_t* hidden, const float* partials, uint32_t splits, const uint16_t* w,
                                   uint16_t* y, uint32_t y_tiled, uint32_t rows, uint32_t width, float eps,
                                   uint32_t* err, hipStream_t s);
hipError_t launch_tile_activation(const uint16_t* x, uint16_t* x_tiled, uint32_t m, uint32_t k, uint32_t to_tiled,
                                  hipStream_t s);
hipError_t launch_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, uint64_t n, uint32_t* err,
                         hipStream_t s);

// projections
// m > kMaxRows: no split-K; n % 128 == 0; x in activation tile order with act_mtiles(m) tiles.
// err receives ERR_NONFINITE from the SwiGLU epilogue (may be null).
hipError_t launch_gemm_large(const uint16_t* x_tiled, const uint16_t* w_tiled, uint32_t m, uint32_t n, uint32_t k,
                             uint32_t epilogue, const uint16_t* residual, void* out, uint32_t ldo, uint32_t* err,
                             hipStream_t s);
// The QKV projection of a prefill chunk with QK-norm, RoPE and the KV
// append fused into its epilogue (qk_head.hpp), q written row-major to
// qa.q_out. Only for the 256 x 256-block kernel: returns
// hipErrorInvalidValue when m <= 256 or n % 256 != 0 (run the projection and
// launch_qknorm_rope_kv instead).
hipError_t launch_gemm_qkv_rope(const uint16_t* x_tiled, const uint16_t* w_tiled, uint32_t m, uint32_t n, uint32_t k,
                                const QkvRopeArgs& qa, hipStream_t s);
hipError_t launch_gemm(const uint16_t* x_tiled, const uint16_t* w_tiled, uint32_t m, uint32_t n, uint32_t k,
                       uint32_t epilogue, uint32_t splits, const uint16_t* residual, void* out, uint32_t ldo,
                       uint32_t* err, hipStream_t s);
// One row's residual + RMSNorm run by every workgroup of the projection that
// consumes it (decode steps of one row): hidden_out = bf16((0 + sum of the
// `splits` slabs of `part`, in split order) + hidden_in) when splits > 0
// (written by one workgroup; hidden_out must not alias hidden_in), then
// x = RMSNorm(hidden) with weight w feeds the projection: the arithmetic and
// order of launch_residual_rmsnorm for that row, bit for bit. splits = 0:
// x = RMSNorm(hidden_in), nothing written.
struct RowNormArgs {
  const uint16_t* hidden_in;
  uint16_t* hidden_out;
  const float* part;  // splits slabs of [slab_rows][width] FP32, row 0 used
  uint32_t splits;
  uint32_t slab_rows;
  const uint16_t* w;
  float eps;
};
// The launch launch_gemm picks for m = 1 (same tiles, splits and summation
// order), with the norm above in the projection's prologue instead of an
// activation operand. Covered: the epilogues PARTIAL (slab counts 0, 4, 6),
// SWIGLU and F32 (4, 6) on the tile shapes these take for the Qwen3 widths,
// k = width in {1024, ..., 4096}, k % 256 == 0; hipErrorInvalidValue
// otherwise.
bool gemm_rownorm_supported(uint32_t n, uint32_t k, uint32_t epilogue, uint32_t splits, uint32_t norm_splits);
hipError_t launch_gemm_rownorm(const uint16_t* w_tiled, uint32_t n, uint32_t k, uint32_t epilogue, uint32_t splits,
                               const RowNormArgs& na, void* out, uint32_t ldo, uint32_t* err, hipStream_t s);
uint32_t gemm_default_splits(uint32_t n, uint32_t k);
// Split-K factor for kMaxRows < m <= kPanelRows (n % kPanelCols == 0).
uint32_t gemm_panel_splits(uint32_t n, uint32_t k);

// attention
// out: [rows][qh*128] row-major, or activation tile order when out_tiled.
// Rows [0, rows) of a launch are rows row0 + [0, rows) of an output of
// out_rows rows (activation tile order with act_mtiles(out_rows) tiles when
// out_tiled, else row-major); q/positions/table/partials are the launch's own.
// Split-context decode attention with split_pages-page partitions (16 or
// 32). partials holds rows x qh x attn_max_splits(context, split_pages)
// records. Rows that fit one partition are finished by the partition launch.
// counters == nullptr: multi-partition rows are finished by
// launch_attention_merge (same split_pages). counters != nullptr: rows x kvh
// words, zero on entry and left zero; the last partition of each (row, KV
// head) to finish merges that pair's records itself, in the same launch.
//
// qkn != nullptr (decode, row0 == 0): the partition kernel also runs the
// QK-norm + RoPE + KV append stage (launch_qknorm_rope_kv's arithmetic, bit
// for bit): every partition forms its query heads from the QKV projection's
// split-K slabs (q is not read), and the partition holding a row's new token
// appends that token's K/V to the caches and uses them. The caller must make
// sure no row reads a slot that another row of the launch writes (each row's
// written page listed by that row only). attention_qkn_supported() gives
// the shapes it covers (at most 4 query heads per KV head, 2 slabs).
struct AttnQkn {
  const float* qkv_part;  // splits slabs of [slab_rows][(qh + 2 kvh) * 128] FP32
  uint32_t splits;
  uint32_t slab_rows;
  const uint16_t* q_norm;
  const uint16_t* k_norm;
  const float* cos_t;  // [context][64]
  const float* sin_t;
  uint16_t* k_cache;  // written: the new token's slot
  uint16_t* v_cache;
  float eps;
};
bool attention_qkn_supported(uint32_t qh, uint32_t kvh, uint32_t qkv_splits);
hipError_t launch_attention_partial(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                    const uint32_t* positions, const uint32_t* table, float* partials, uint16_t* out,
                                    uint32_t out_tiled, uint32_t row0, uint32_t out_rows, uint32_t rows, uint32_t qh,
                                    uint32_t kvh, uint32_t stride, uint32_t pages, uint32_t context,
                                    uint32_t split_pages, uint32_t* counters, uint32_t* err, hipStream_t s,
                                    const AttnQkn* qkn = nullptr);
hipError_t launch_attention_merge(const float* partials, const uint32_t* positions, uint16_t* out,
                                  uint32_t out_tiled, uint32_t row0, uint32_t out_rows, uint32_t rows, uint32_t qh,
                                  uint32_t context, uint32_t split_pages, uint32_t* err, hipStream_t s);

// Prefill attention over blocks of consecutive rows of one sequence (see
// k_attention_block.hip). blocks[i] = first row | (rows << 16); each block
// has at most attention_block_rows(qh, kvh) rows at consecutive positions,
// and its last row's page table serves all of them. No scratch, no merge.
// qkn != nullptr: the QK-norm, RoPE and KV append of every block row run in
// the attention workgroups (AttnQkn as for the decode partitions; q unused).
// The caller guarantees that no block's pages hold a slot another block of
// the launch writes.
uint32_t attention_block_rows(uint32_t qh, uint32_t kvh);
bool attention_blocks_qkn_supported(uint32_t qh, uint32_t kvh, uint32_t qkv_splits);
hipError_t launch_attention_blocks(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                   const uint32_t* positions, const uint32_t* table, const uint32_t* blocks,
                                   uint32_t nblocks, uint16_t* out, uint32_t out_tiled, uint32_t out_rows,
                                   uint32_t qh, uint32_t kvh, uint32_t stride, uint32_t pages, uint32_t context,
                                   uint32_t* err, hipStream_t s, const AttnQkn* qkn = nullptr);

// logits
// With host_choices (coherent pinned memory), the choices and the error word
// (at host_err) are also stored there, so the host reads them without a
// device-to-host copy; with host_done, row r's word is then set to 1 with a
// system-scope release (row 0's after the error word too), so a host that
// sees every row's word set reads complete choices and error bits.
hipError_t launch_argmax(const float* logits, uint32_t rows, uint32_t vocab, void* scratch, uint32_t* choices,
                         uint32_t* err, hipStream_t s, uint32_t* host_choices = nullptr, uint32_t* host_err = nullptr,
                         uint32_t* host_done = nullptr);

}  // namespace fh
