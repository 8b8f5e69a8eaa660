// C ABI for the individual kernel roots (fh_op_*), scratch sizing, and the
// integer speculative-decoding helpers. Every entry point validates its
// shapes on the host before launching, so a kernel never sees a geometry it
// was not written for.
#include <cstring>
#include <mutex>

#include "../../include/ferric_hip.h"
#include "kernels.hpp"

namespace {

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline fh_status status_of(hipError_t e) {
  if (e == hipSuccess) return FH_OK;
  fh::set_thread_error(hipGetErrorString(e));
  return FH_ERR_DEVICE;
}

// Launchers report hipGetLastError(), which also returns an error left
// behind by an unrelated earlier runtime call on this thread; clear it first
// so that the status belongs to this launch.
#define from_hip(expr) (static_cast<void>(hipGetLastError()), status_of(expr))

}  // namespace

extern "C" {

fh_status fh_op_tile_weight(const uint16_t* src, uint16_t* dst, uint32_t n, uint32_t k, void* stream) {
  if (!src || !dst || n == 0 || k == 0 || n % 16 || k % 32) return FH_ERR_INVALID_ARGUMENT;
  return from_hip(fh::launch_tile_weight(src, dst, n, k, 1, 0, as_stream(stream)));
}

fh_status fh_op_tile_gate_up(const uint16_t* gate, const uint16_t* up, uint16_t* dst, uint32_t i, uint32_t k,
                             void* stream) {
  if (!gate || !up || !dst || i == 0 || k == 0 || i % 16 || k % 32) return FH_ERR_INVALID_ARGUMENT;
  (void)hipGetLastError();
  hipError_t e = fh::launch_tile_weight(gate, dst, i, k, 2, 0, as_stream(stream));
  if (e == hipSuccess) e = fh::launch_tile_weight(up, dst, i, k, 2, 1, as_stream(stream));
  return status_of(e);
}

fh_status fh_op_untile_weight(const uint16_t* tiled, uint16_t* dst, uint32_t n, uint32_t k, void* stream) {
  if (!tiled || !dst || n == 0 || k == 0 || n % 16 || k % 32) return FH_ERR_INVALID_ARGUMENT;
  return from_hip(fh::launch_untile_weight(tiled, dst, n, k, as_stream(stream)));
}

fh_status fh_op_embedding(const uint32_t* tokens, const uint16_t* table_tiled, uint16_t* out, uint32_t rows,
                          uint32_t hidden, uint32_t vocabulary, uint32_t* error_word, void* stream) {
  if (!tokens || !table_tiled || !out || rows == 0 || hidden == 0 || hidden % 32 || vocabulary == 0 ||
      vocabulary % 16)
    return FH_ERR_INVALID_ARGUMENT;
  return from_hip(fh::launch_embedding(tokens, table_tiled, out, rows, hidden, vocabulary, error_word,
                                       as_stream(stream)));
}

fh_status fh_op_rmsnorm(const uint16_t* x, const uint16_t* weight, uint16_t* y, uint32_t rows, uint32_t width,
                        float epsilon, uint32_t* error_word, void* stream) {
  if (!x || !weight || !y || rows == 0 || width == 0 || width % 8 || width > 8192) return FH_ERR_INVALID_ARGUMENT;
  return from_hip(fh::launch_rmsnorm(x, weight, y, rows, width, epsilon, error_word, as_stream(stream)));
}

fh_status fh_op_gemm(const uint16_t* x_tiled, const uint16_t* w_tiled, uint32_t m, uint32_t n, uint32_t k,
                     uint32_t epilogue, uint32_t splits, const uint16_t* residual, void* out, uint32_t ldo,
                     uint32_t* error_word, void* stream) {
  if (!x_tiled || !w_tiled || !out || m == 0 || n == 0 || k == 0 || n % 16 || k % 32) return FH_ERR_INVALID_ARGUMENT;
  if (epilogue > FH_EPI_PARTIAL || splits == 0 || splits > k / 32) return FH_ERR_INVALID_ARGUMENT;
  if (epilogue != FH_EPI_PARTIAL && splits != 1) return FH_ERR_INVALID_ARGUMENT;
  if (epilogue == FH_EPI_RESIDUAL && !residual) return FH_ERR_INVALID_ARGUMENT;
  if (epilogue == FH_EPI_SWIGLU) {
    if (n % 32) return FH_ERR_INVALID_ARGUMENT;  // the output is in activation tile order
  } else if (ldo < n) {
    return FH_ERR_INVALID_ARGUMENT;
  }
  if (m > fh::kMaxRows) {
    // Wide and prefill-size batches: n % 128 == 0, 16-byte aligned FP32 rows
    // (8-byte bf16 rows); split-K partials up to kPanelRows rows.
    if (n % fh::kPanelCols || (epilogue != FH_EPI_SWIGLU && ldo % 4)) return FH_ERR_INVALID_ARGUMENT;
    if (epilogue == FH_EPI_PARTIAL) {
      if (!fh::gemm_partial_rows_ok(m, n)) return FH_ERR_INVALID_ARGUMENT;
      return from_hip(fh::launch_gemm(x_tiled, w_tiled, m, n, k, epilogue, splits, residual, out, ldo, error_word,
                                      as_stream(stream)));
    }
    return from_hip(fh::launch_gemm_large(x_tiled, w_tiled, m, n, k, epilogue, residual, out, ldo, error_word,
                                                  as_stream(stream)));
  }
  return from_hip(fh::launch_gemm(x_tiled, w_tiled, m, n, k, epilogue, splits, residual, out, ldo, error_word,
                                            as_stream(stream)));
}

uint32_t fh_activation_rows(uint32_t m) { return m ? fh::act_mtiles(m) * 16 : 0u; }

uint32_t fh_gemm_default_splits(uint32_t n, uint32_t k) { return fh::gemm_default_splits(n, k); }

uint32_t fh_partial_slab_rows(uint32_t m) { return m == 0 || m > fh::kPanelRows ? 0u : fh::partial_slab_rows(m); }

fh_status fh_op_tile_activation(const uint16_t* x, uint16_t* x_tiled, uint32_t m, uint32_t k, void* stream) {
  if (!x || !x_tiled || m == 0 || k == 0 || k % 32) return FH_ERR_INVALID_ARGUMENT;
  return from_hip(fh::launch_tile_activation(x, x_tiled, m, k, 1, as_stream(stream)));
}

fh_status fh_op_untile_activation(const uint16_t* x_tiled, uint16_t* x, uint32_t m, uint32_t k, void* stream) {
  if (!x || !x_tiled || m == 0 || k == 0 || k % 32) return FH_ERR_INVALID_ARGUMENT;
  return from_hip(fh::launch_tile_activation(x, const_cast<uint16_t*>(x_tiled), m, k, 0, as_stream(stream)));
}

fh_status fh_op_residual_rmsnorm(uint16_t* hidden, const float* partials, uint32_t splits, const uint16_t* weight,
                                 uint16_t* y, uint32_t y_tiled, uint32_t rows, uint32_t width, float epsilon,
                                 uint32_t* error_word, void* stream) {
  if (!hidden || !weight || !y || rows == 0 || width == 0 || width % 32 || width > 8192 || (splits && !partials))
    return FH_ERR_INVALID_ARGUMENT;
  if (splits && rows > fh::kPanelRows) return FH_ERR_INVALID_ARGUMENT;
  return from_hip(fh::launch_residual_rmsnorm(hidden, partials, splits, weight, y, y_tiled, rows, width, epsilon,
                                              error_word, as_stream(stream)));
}

fh_status fh_op_gemm_rmsnorm(const uint16_t* hidden_in, uint16_t* hidden_out, const float* partials,
                             uint32_t norm_splits, const uint16_t* norm_weight, float epsilon,
                             const uint16_t* w_tiled, uint32_t n, uint32_t k, uint32_t epilogue, uint32_t splits,
                             void* out, uint32_t ldo, uint32_t* error_word, void* stream) {
  if (!hidden_in || !norm_weight || !w_tiled || !out || n == 0 || n % 16) return FH_ERR_INVALID_ARGUMENT;
  if (norm_splits && (!partials || !hidden_out || hidden_out == hidden_in)) return FH_ERR_INVALID_ARGUMENT;
  if (epilogue != FH_EPI_SWIGLU && ldo < n) return FH_ERR_INVALID_ARGUMENT;
  if (!fh::gemm_rownorm_supported(n, k, epilogue, splits, norm_splits)) return FH_ERR_INVALID_ARGUMENT;
  fh::RowNormArgs na{hidden_in, hidden_out, partials, norm_splits, fh::partial_slab_rows(1), norm_weight, epsilon};
  return from_hip(fh::launch_gemm_rownorm(w_tiled, n, k, epilogue, splits, na, out, ldo, error_word,
                                          as_stream(stream)));
}

uint32_t fh_gemm_rmsnorm_supported(uint32_t n, uint32_t k, uint32_t epilogue, uint32_t splits, uint32_t norm_splits) {
  return n && n % 16 == 0 && fh::gemm_rownorm_supported(n, k, epilogue, splits, norm_splits) ? 1u : 0u;
}

fh_status fh_op_qknorm_rope_kv(const void* qkv, uint32_t qkv_splits, const uint16_t* q_norm, const uint16_t* k_norm,
                               const float* cos_table, const float* sin_table, const uint32_t* positions,
                               const uint32_t* page_table, uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
                               uint32_t rows, uint32_t query_heads, uint32_t kv_heads, uint32_t stride,
                               uint32_t physical_pages, uint32_t context_tokens, float epsilon, uint32_t* error_word,
                               void* stream) {
  if (!qkv || !q_norm || !k_norm || !cos_table || !sin_table || !positions || !page_table || !q_out || !k_cache ||
      !v_cache || rows == 0 || query_heads == 0 || kv_heads == 0 || query_heads + 2 * kv_heads > 64 || stride == 0 ||
      physical_pages == 0 || context_tokens == 0 || (qkv_splits && rows > fh::kPanelRows))
    return FH_ERR_INVALID_ARGUMENT;
  const uint16_t* bf = qkv_splits ? nullptr : reinterpret_cast<const uint16_t*>(qkv);
  const float* part = qkv_splits ? reinterpret_cast<const float*>(qkv) : nullptr;
  return from_hip(fh::launch_qknorm_rope_kv(bf, part, qkv_splits, q_norm, k_norm, cos_table, sin_table, positions,
                                            page_table, q_out, k_cache, v_cache, rows, query_heads, kv_heads, stride,
                                            physical_pages, context_tokens, epsilon, error_word, as_stream(stream)));
}

}  // extern "C"

// ---- no-allocation attention ----------------------------------------------
// fh_op_paged_attention_noalloc keeps its partition records in this
// file-scope device array instead of a caller workspace. In host code
// `g_noalloc_attn_records` is only a stand-in symbol: its device address is
// resolved once per device (hipGetSymbolAddress, with that device current)
// and only that address is ever handed to kernels. Every call on a GPU shares the GPU's
// copy, so calls that overlap on one GPU race; each call writes every record
// it later reads, so nothing needs clearing between calls.
namespace {
constexpr uint64_t kNoAllocAttnRecords = 16384;  // rows x query heads x partitions (8.5 MB)
constexpr int kNoAllocMaxDevices = 64;
std::mutex g_records_mu;
void* g_records_dev[kNoAllocMaxDevices] = {};
}  // namespace

static __device__ __align__(256) float g_noalloc_attn_records[kNoAllocAttnRecords * fh::kAttnPartialFloats];

namespace {
// The device address of `g_noalloc_attn_records` on the stream's device (NULL
// and an error message on failure).
float* noalloc_records(hipStream_t s) {
  int dev = -1;
  hipError_t e = s ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kNoAllocMaxDevices) {
    fh::set_thread_error(e != hipSuccess ? hipGetErrorString(e) : "device ordinal out of range");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_records_mu);
  if (!g_records_dev[dev]) {
    int cur = -1;
    e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
    void* ptr = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(g_noalloc_attn_records));
    if (cur >= 0 && cur != dev) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess || !ptr) {
      fh::set_thread_error(e != hipSuccess ? hipGetErrorString(e) : "no device address for the record array");
      return nullptr;
    }
    g_records_dev[dev] = ptr;
  }
  return reinterpret_cast<float*>(g_records_dev[dev]);
}
}  // namespace

extern "C" {

fh_status fh_op_paged_attention_noalloc(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                        const uint32_t* positions, const uint32_t* page_table, uint16_t* out,
                                        uint32_t out_tiled, uint32_t rows, uint32_t query_heads, uint32_t kv_heads,
                                        uint32_t stride, uint32_t physical_pages, uint32_t context_tokens,
                                        uint32_t* error_word, void* stream) {
  if (!q || !k_cache || !v_cache || !positions || !page_table || !out || rows == 0 || kv_heads == 0 ||
      query_heads % kv_heads != 0 || stride == 0 || physical_pages == 0 || context_tokens == 0 ||
      (uint64_t)stride * 16 < context_tokens)
    return FH_ERR_INVALID_ARGUMENT;
  const uint32_t g = query_heads / kv_heads;
  if (g != 1 && g != 2 && g != 4 && g != 8) return FH_ERR_INVALID_ARGUMENT;
  const uint32_t split_pages = fh::attn_split_pages(rows, query_heads, context_tokens);
  const uint64_t records = (uint64_t)rows * query_heads * fh::attn_max_splits(context_tokens, split_pages);
  if (records > kNoAllocAttnRecords) {
    fh::set_thread_error("fh_op_paged_attention_noalloc: rows x query_heads x partitions of the context exceeds "
                         "the 16384 partition records of its static array");
    return FH_ERR_INVALID_ARGUMENT;
  }
  hipStream_t s = as_stream(stream);
  float* part = noalloc_records(s);
  if (!part) return FH_ERR_DEVICE;
  (void)hipGetLastError();
  hipError_t e = fh::launch_attention_partial(q, k_cache, v_cache, positions, page_table, part, out, out_tiled, 0,
                                              rows, rows, query_heads, kv_heads, stride, physical_pages,
                                              context_tokens, split_pages, nullptr, error_word, s);
  if (e == hipSuccess)
    e = fh::launch_attention_merge(part, positions, out, out_tiled, 0, rows, rows, query_heads, context_tokens,
                                   split_pages, error_word, s);
  return status_of(e);
}

uint64_t fh_attention_scratch_bytes(uint32_t rows, uint32_t query_heads, uint32_t context_tokens) {
  return (uint64_t)rows * query_heads *
         fh::attn_max_splits(context_tokens, fh::attn_split_pages(rows, query_heads, context_tokens)) * fh::kAttnPartialFloats * 4;
}

fh_status fh_op_qknorm_paged_attention(const float* qkv_partials, uint32_t qkv_splits, const uint16_t* q_norm,
                                       const uint16_t* k_norm, const float* cos_table, const float* sin_table,
                                       const uint32_t* positions, const uint32_t* page_table, uint16_t* k_cache,
                                       uint16_t* v_cache, uint16_t* out, uint32_t out_tiled, void* scratch,
                                       uint32_t rows, uint32_t query_heads, uint32_t kv_heads, uint32_t stride,
                                       uint32_t physical_pages, uint32_t context_tokens, float epsilon,
                                       uint32_t* error_word, void* stream) {
  if (!qkv_partials || !q_norm || !k_norm || !cos_table || !sin_table || !positions || !page_table || !k_cache ||
      !v_cache || !out || !scratch || rows == 0 || rows > fh::kMaxRows || stride == 0 || physical_pages == 0 ||
      context_tokens == 0 || (uint64_t)stride * 16 < context_tokens ||
      !fh::attention_qkn_supported(query_heads, kv_heads, qkv_splits))
    return FH_ERR_INVALID_ARGUMENT;
  hipStream_t s = as_stream(stream);
  float* part = reinterpret_cast<float*>(scratch);
  const uint32_t split_pages = fh::attn_split_pages(rows, query_heads, context_tokens);
  const fh::AttnQkn qa{qkv_partials, qkv_splits, fh::partial_slab_rows(rows), q_norm, k_norm, cos_table, sin_table,
                       k_cache,      v_cache,    epsilon};
  (void)hipGetLastError();
  hipError_t e = fh::launch_attention_partial(nullptr, k_cache, v_cache, positions, page_table, part, out, out_tiled,
                                              0, rows, rows, query_heads, kv_heads, stride, physical_pages,
                                              context_tokens, split_pages, nullptr, error_word, s, &qa);
  if (e == hipSuccess)
    e = fh::launch_attention_merge(part, positions, out, out_tiled, 0, rows, rows, query_heads, context_tokens,
                                   split_pages, error_word, s);
  return status_of(e);
}

fh_status fh_op_paged_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                const uint32_t* positions, const uint32_t* page_table, uint16_t* out,
                                uint32_t out_tiled, void* scratch, uint32_t rows, uint32_t query_heads,
                                uint32_t kv_heads, uint32_t stride, uint32_t physical_pages, uint32_t context_tokens,
                                uint32_t* error_word, void* stream) {
  if (!q || !k_cache || !v_cache || !positions || !page_table || !out || !scratch || rows == 0 || kv_heads == 0 ||
      query_heads % kv_heads != 0 || stride == 0 || physical_pages == 0 || context_tokens == 0 ||
      (uint64_t)stride * 16 < context_tokens)
    return FH_ERR_INVALID_ARGUMENT;
  const uint32_t g = query_heads / kv_heads;
  if (g != 1 && g != 2 && g != 4 && g != 8) return FH_ERR_INVALID_ARGUMENT;
  hipStream_t s = as_stream(stream);
  float* part = reinterpret_cast<float*>(scratch);
  const uint32_t split_pages = fh::attn_split_pages(rows, query_heads, context_tokens);
  (void)hipGetLastError();
  hipError_t e = fh::launch_attention_partial(q, k_cache, v_cache, positions, page_table, part, out, out_tiled, 0,
                                              rows, rows, query_heads, kv_heads, stride, physical_pages,
                                              context_tokens, split_pages, nullptr, error_word, s);
  if (e == hipSuccess)
    e = fh::launch_attention_merge(part, positions, out, out_tiled, 0, rows, rows, query_heads, context_tokens,
                                   split_pages, error_word, s);
  return status_of(e);
}

fh_status fh_op_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, uint64_t elements,
                       uint32_t* error_word, void* stream) {
  if (!gate || !up || !out || elements == 0) return FH_ERR_INVALID_ARGUMENT;
  return from_hip(fh::launch_swiglu(gate, up, out, elements, error_word, as_stream(stream)));
}

uint64_t fh_argmax_scratch_bytes(uint32_t rows) { return (uint64_t)rows * fh::kArgmaxShards * 8; }

fh_status fh_op_argmax(const float* logits, uint32_t rows, uint32_t vocabulary, void* scratch, uint32_t* choices,
                       uint32_t* error_word, void* stream) {
  if (!logits || !scratch || !choices || rows == 0 || vocabulary == 0) return FH_ERR_INVALID_ARGUMENT;
  return from_hip(fh::launch_argmax(logits, rows, vocabulary, scratch, choices, error_word, as_stream(stream)));
}

fh_status fh_op_synth_fill(uint16_t* dst, uint64_t count, uint64_t tensor_seed, float scale, void* stream) {
  if (!dst || count == 0) return FH_ERR_INVALID_ARGUMENT;
  return from_hip(fh::launch_synth_fill(dst, count, tensor_seed, scale, as_stream(stream)));
}

// target_ids[s][0] = anchor, target_ids[s][1 + i] = draft[i][s]
// (ferric_qwen3_speculative_token_assembly_v1, device/qwen3-all-kernels-v1/src/logits.rs:587).
fh_status fh_speculative_token_assembly(const uint32_t* anchors, const uint32_t* draft, uint32_t sequences,
                                        uint32_t k, uint32_t* target_ids) {
  if (!anchors || (k && !draft) || !target_ids || sequences == 0) return FH_ERR_INVALID_ARGUMENT;
  for (uint32_t s = 0; s < sequences; ++s) {
    target_ids[(uint64_t)s * (k + 1)] = anchors[s];
    for (uint32_t i = 0; i < k; ++i) target_ids[(uint64_t)s * (k + 1) + 1 + i] = draft[(uint64_t)i * sequences + s];
  }
  return FH_OK;
}

// Per-sequence completion record of ferric_qwen3_compact_completion_v1
// (device/qwen3-all-kernels-v1/src/logits.rs:279-520), 120 bytes little-endian:
//   [0,4) request slot  [4,8) request generation  [8,16) completion epoch
//   [16,48) plan identity  [48] accepted  [49] emitted = accepted + 1  [50,52) 0
//   [52,120) emitted tokens (draft[0..accepted) then the correction), then zeros.
// A sequence with live length 0 gets an all-zero record and is not checked
// further. The checks are the reference kernel's traps, in its order: live
// <= active_tokens (and, speculative, live == active_tokens), slot < 32,
// generation != 0, a nonzero plan identity, then each compared (draft, target)
// pair below the vocabulary up to and including the first mismatch (tokens
// after it are never read), then the correction token. The reference admits
// a fixed profile table (logits.rs:293-304); this entry point accepts any
// 1..32 sequences (its grid bound), active_tokens >= 1 and K <= 16 with
// active_tokens = K + 1, which includes the 32-sequence K = 4 rounds the
// reference's table stops short of. Nothing is written unless every
// sequence passes.
namespace {
constexpr uint32_t kRecordBytes = 120;
constexpr uint32_t kQwen3Vocabulary = 151936;  // QWEN3_LOGITS_VOCABULARY_V1, logits.rs:22
constexpr uint32_t kMaxSpeculativeK = 16;       // QWEN3_LOGITS_MAX_SPECULATIVE_K_V1
constexpr uint32_t kMaxSequences = 32;          // QWEN3_LOGITS_COMPACT_MAX_GRID_WORKGROUPS_V1

void put_le(uint8_t* dst, uint64_t v, int bytes) {
  for (int i = 0; i < bytes; ++i) dst[i] = (uint8_t)(v >> (8 * i));
}

bool one_record(const uint32_t* choices, const uint32_t* draft, uint32_t live, uint32_t slot, uint32_t generation,
                uint64_t epoch, const uint8_t* plan, uint32_t sequences, uint32_t sequence, uint32_t active_tokens,
                uint32_t k, uint8_t* rec) {
  std::memset(rec, 0, kRecordBytes);
  if (live == 0) return true;
  if (live > active_tokens || (k != 0 && live != active_tokens)) return false;
  if (slot >= 32 || generation == 0) return false;
  bool plan_present = false;
  for (int b = 0; b < 32; ++b) plan_present |= plan[b] != 0;
  if (!plan_present) return false;
  const uint64_t base = (uint64_t)sequence * active_tokens;
  uint32_t accepted = 0;
  while (accepted < k) {
    const uint32_t d = draft[(uint64_t)accepted * sequences + sequence];
    const uint32_t t = choices[base + accepted];
    if (d >= kQwen3Vocabulary || t >= kQwen3Vocabulary) return false;
    if (d != t) break;
    ++accepted;
  }
  if (accepted >= active_tokens) return false;
  const uint32_t correction = choices[base + (k == 0 ? live - 1 : accepted)];
  if (correction >= kQwen3Vocabulary) return false;
  put_le(rec + 0, slot, 4);
  put_le(rec + 4, generation, 4);
  put_le(rec + 8, epoch, 8);
  std::memcpy(rec + 16, plan, 32);
  rec[48] = (uint8_t)accepted;
  rec[49] = (uint8_t)(accepted + 1);
  for (uint32_t i = 0; i < accepted; ++i) put_le(rec + 52 + 4 * i, draft[(uint64_t)i * sequences + sequence], 4);
  put_le(rec + 52 + 4 * accepted, correction, 4);
  return true;
}
}  // namespace

fh_status fh_compact_completion(const uint32_t* choices, const uint32_t* draft, const uint32_t* active_lengths,
                                const uint32_t* request_slots, const uint32_t* request_generations,
                                const uint64_t* completion_epochs, const uint8_t* plan_identities, uint32_t sequences,
                                uint32_t active_tokens, uint32_t speculative_k, uint8_t* records) {
  if (!choices || !active_lengths || !request_slots || !request_generations || !completion_epochs ||
      !plan_identities || !records || sequences == 0 || sequences > kMaxSequences || active_tokens == 0 ||
      speculative_k > kMaxSpeculativeK || (speculative_k != 0 && (!draft || active_tokens != speculative_k + 1))) {
    fh::set_thread_error("compact completion: bad geometry");
    return FH_ERR_INVALID_ARGUMENT;
  }
  uint8_t out[kMaxSequences * kRecordBytes];
  for (uint32_t s = 0; s < sequences; ++s) {
    if (!one_record(choices, draft, active_lengths[s], request_slots[s], request_generations[s],
                    completion_epochs[s], plan_identities + 32ull * s, sequences, s, active_tokens, speculative_k,
                    out + (uint64_t)s * kRecordBytes)) {
      fh::set_thread_error("compact completion: a sequence's request, plan or tokens were rejected");
      return FH_ERR_INVALID_ARGUMENT;
    }
  }
  std::memcpy(records, out, (uint64_t)sequences * kRecordBytes);
  return FH_OK;
}

// Greedy speculative verification (crates/ferric-spec/src/speculation.rs:126-200).
fh_status fh_verify_greedy_round(const uint32_t* draft, uint32_t draft_count, const uint32_t* target,
                                 uint32_t target_count, uint32_t* accepted, uint32_t* emitted,
                                 uint32_t* emitted_count) {
  if (!target || !accepted || !emitted || !emitted_count || (draft_count && !draft)) return FH_ERR_INVALID_ARGUMENT;
  if (target_count == 0) return FH_ERR_INVALID_ARGUMENT;                  // MissingTargetBonus
  if (draft_count == 0xffffffffu) return FH_ERR_INVALID_ARGUMENT;         // DraftTokenCountOverflow
  if (target_count != draft_count + 1) return FH_ERR_INVALID_ARGUMENT;    // IncorrectTargetChoiceCount
  uint32_t a = 0;
  while (a < draft_count && draft[a] == target[a]) ++a;
  for (uint32_t i = 0; i < a; ++i) emitted[i] = draft[i];
  emitted[a] = target[a];
  *accepted = a;
  *emitted_count = a + 1;
  return FH_OK;
}

fh_status fh_verify_greedy_batch(const uint32_t* draft, const uint32_t* target, uint32_t sequences, uint32_t k,
                                 uint32_t* accepted, uint32_t* emitted) {
  if (sequences == 0) return FH_OK;
  if (!target || !accepted || !emitted || (k && !draft)) return FH_ERR_INVALID_ARGUMENT;
  if (k == 0xffffffffu) return FH_ERR_INVALID_ARGUMENT;  // DraftTokenCountOverflow
  const uint64_t stride = (uint64_t)k + 1;
  for (uint32_t s = 0; s < sequences; ++s) {
    const uint32_t* t = target + s * stride;
    uint32_t* e = emitted + s * stride;
    uint32_t a = 0;
    while (a < k && draft[(uint64_t)a * sequences + s] == t[a]) ++a;
    for (uint32_t i = 0; i < a; ++i) e[i] = draft[(uint64_t)i * sequences + s];
    e[a] = t[a];
    accepted[s] = a;
  }
  return FH_OK;
}

}  // extern "C"
