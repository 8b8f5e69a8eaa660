// Host runtime behind the C ABI: the resident model (weights in MFMA tile
// order), the paged KV pool, per-step metadata, and fh_execute_batch — the
// replacement for EngineeringTpBatchExecutionV2::forward
// (adapters/m1-engineering-execution-v1/src/tp_execution/batched.rs:1746-2454).
//
// One decode step = 5 + (7, 8 or 9) x layers kernel launches (one row:
// 4 + (5, 6 or 7) x layers, the norms inside the projections) on one HIP
// stream (enqueue_step; fh_expected_dispatch_count counts the same code
// without launching), optionally replayed from a HIP graph captured once per
// row count and attention form. All per-step inputs
// (tokens, positions, page tables) live in one device block that the step's
// first launch refreshes from a coherent pinned host block, and the last
// launch stores the choices and error word into another, so a captured
// graph stays valid across steps and a step needs no copy beside it.
// Prefill chunks (run_prefill) keep a host-to-device copy of their metadata.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/ferric_hip.h"
#include "../../include/ferric_synth.h"
#include "common.hpp"
#include "kernels.hpp"

namespace {

constexpr uint32_t kNoLayer = 0xffffffffu;  // QWEN3_NO_LAYER, crates/ferric-spec/src/qwen3.rs:12
constexpr uint32_t kPageTokens = 16;
constexpr uint32_t kMaxRows = 32;
// Prefill chunks: attention runs over this many rows per launch pair (bounds
// the partition-state scratch), and at most this many output rows get logits.
constexpr uint32_t kMaxPrefillOutputs = 256;

thread_local std::string g_create_error;

struct LayerWeights {
  uint16_t* qkv = nullptr;   // tiled [(qh + 2 kvh) * 128][hidden]
  uint16_t* o = nullptr;     // tiled [hidden][qh * 128]
  uint16_t* gu = nullptr;    // tiled, gate/up interleaved by tile [2 * inter][hidden]
  uint16_t* down = nullptr;  // tiled [hidden][inter]
  uint16_t* in_norm = nullptr;
  uint16_t* post_norm = nullptr;
  uint16_t* q_norm = nullptr;
  uint16_t* k_norm = nullptr;
};

struct ProfiledLaunch {
  uint32_t cls;
  hipEvent_t begin, end;
};

}  // namespace

struct fh_ctx {
  fh_model_desc md{};
  fh_ctx_options opt{};
  hipStream_t stream = nullptr;
  std::vector<void*> device_allocs;
  std::vector<void*> host_allocs;

  std::vector<LayerWeights> layers;
  uint16_t* embed = nullptr;  // tiled [vocab][hidden]
  uint16_t* head = nullptr;   // tiled [vocab][hidden] (== embed when tied)
  uint16_t* final_norm = nullptr;
  uint16_t* staging = nullptr;  // row-major upload/synthesis buffer
  uint64_t staging_elems = 0;

  uint16_t* kv = nullptr;
  uint64_t kv_slab_elems = 0;  // one K or V cache of one layer: pages * 16 * kvh * 128

  float* cos_t = nullptr;
  float* sin_t = nullptr;

  uint16_t* hidden = nullptr;  // residual stream, row-major [cap][hidden]
  uint16_t* hidden_alt = nullptr;  // one row: the residual stream's other buffer in one-row steps
  bool row_norm_fused = false;     // one-row steps run each norm in the consuming projection
  uint16_t* xn = nullptr;      // normalized rows, activation tile order
  uint16_t* qrot = nullptr;    // rotated queries, row-major [cap][qh*128]
  uint16_t* attn = nullptr;    // attention output, activation tile order
  uint16_t* act = nullptr;     // SwiGLU output, activation tile order
  float* qkv_part = nullptr;   // split-K partial slabs [s_qkv][32][nqkv]
  float* o_part = nullptr;     // [s_o][32][hidden]
  float* down_part = nullptr;  // [s_down][32][hidden]
  uint32_t s_qkv = 1, s_o = 1, s_down = 1;
  float* logits = nullptr;
  float* attn_part = nullptr;
  uint32_t* attn_count = nullptr;  // [cap][kvh] partition arrival counters, zero between launches
  void* argmax_scratch = nullptr;
  uint32_t* choices = nullptr;
  uint32_t* err = nullptr;
  uint16_t* capture = nullptr;  // [layers][capture_rows][hidden]: residual stream after each layer
  uint32_t capture_rows = 0;    // max(row_capacity, prefill_rows)

  uint32_t* d_meta = nullptr;  // tokens[cap] | positions[cap] | table[cap][stride]
  uint32_t* h_meta = nullptr;  // pinned mirror
  uint32_t* h_out = nullptr;   // pinned: choices[cap] | error word | done[cap] (one word per row)

  // Prefill chunks (row_capacity < rows <= prefill_rows); allocated only when
  // prefill_rows > 0. Activation-tile buffers hold act_mtiles(prefill_rows) tiles.
  struct Prefill {
    uint16_t* hidden = nullptr;    // [rows][hidden]
    uint16_t* xn = nullptr;        // tiled
    uint16_t* qkv = nullptr;       // [rows][nqkv]
    uint16_t* qrot = nullptr;      // [rows][qh*128]
    uint16_t* attn = nullptr;      // tiled
    uint16_t* act = nullptr;       // tiled
    uint16_t* out_hidden = nullptr;  // gathered output rows [kMaxPrefillOutputs][hidden]
    uint16_t* out_xn = nullptr;    // tiled
    // Split-K partial slabs of chunks of up to kPanelRows rows, shared by the
    // QKV, O and down projections of a layer (each consumed before the next
    // is written): [splits][partial_slab_rows(rows)][n].
    float* part = nullptr;
    uint32_t s_qkv = 1, s_o = 1, s_down = 1;  // splits for kMaxRows < rows <= kPanelRows
    float* logits = nullptr;       // [kMaxPrefillOutputs][vocab]
    void* argmax_scratch = nullptr;
    uint32_t* choices = nullptr;
    uint32_t* d_meta = nullptr;    // tokens[P] | positions[P] | output rows[kMaxPrefillOutputs] | blocks[P] | table[P][stride]
    uint32_t* h_meta = nullptr;
    uint32_t* h_out = nullptr;     // choices[kMaxPrefillOutputs] | error word
  } pre;
  const float* last_logits = nullptr;  // what fh_read_logits copies
  bool last_was_prefill = false;
  std::string launch_detail;  // which launch failed first in the last enqueue

  uint32_t nqkv = 0;
  std::vector<uint8_t> have;  // which tensors are resident
  bool poisoned = false;
  uint64_t last_batch = 0;
  uint64_t dispatches = 0;
  uint32_t last_rows = 0;        // rows with logits in the last batch (output rows for prefill)
  uint32_t last_batch_rows = 0;  // token rows of the last batch
  std::string error;

  // One captured decode step per row count and attention form, with the
  // number of launches the capture recorded (what a replay issues).
  struct StepGraph {
    hipGraphExec_t exec = nullptr;
    uint64_t launches = 0;
  };
  std::map<uint32_t, StepGraph> graphs;
  std::vector<hipGraph_t> graph_defs;
  hipEvent_t ev_begin = nullptr, ev_end = nullptr;
  float last_ms = 0.f;

  bool profiling = false;
  std::vector<hipEvent_t> prof_events;
  std::vector<ProfiledLaunch> prof_launches;
  float class_ms[FH_KC_COUNT] = {};
  uint32_t class_launches[FH_KC_COUNT] = {};

  // Validation scratch (stamped arrays, sized by physical_pages).
  // Batch validation: per physical page, the batch that last listed it
  // (stamp), the owner (sequence, logical index) that batch gave it, whether
  // two owners disagree, and the last row that listed it.
  struct PageOwner {
    uint64_t stamp = 0;
    uint64_t sequence = 0;
    uint32_t logical = 0;
    uint32_t row = 0;
    uint32_t conflict = 0;
    uint32_t multi = 0;  // listed by more than one row of the batch
  };
  std::vector<PageOwner> page_owner;
  std::vector<uint8_t> row_dup;  // per row of the batch: a page listed twice
  bool batch_private_slots = false;  // no row lists a page another row of the batch writes
  bool last_qkn = false;             // the last decode step ran QK-norm/KV append inside attention
  std::vector<uint64_t> slot_scratch;
  uint64_t stamp = 0;
};

namespace {

fh_status fail(fh_ctx* ctx, fh_status st, const std::string& msg) {
  if (ctx)
    ctx->error = msg;
  else
    g_create_error = msg;
  return st;
}

fh_status hip_fail(fh_ctx* ctx, hipError_t e, const char* what) {
  return fail(ctx, FH_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

#define FH_HIP(ctx, expr)                                  \
  do {                                                     \
    hipError_t e_ = (expr);                                \
    if (e_ != hipSuccess) return hip_fail(ctx, e_, #expr); \
  } while (0)

uint32_t tensor_index(uint32_t kind, uint32_t layer, uint32_t layers) {
  // Globals first (head, embedding, final norm), then 11 per layer.
  if (kind <= FH_FINAL_NORM) return kind;
  return 3 + layer * 11 + (kind - FH_INPUT_LAYER_NORM);
}

bool is_global(uint32_t kind) { return kind <= FH_FINAL_NORM; }

// Rows x columns of each tensor (norms: 1 x width).
bool tensor_shape(const fh_model_desc& md, uint32_t kind, uint64_t* rows, uint64_t* cols) {
  const uint64_t h = md.hidden, q = (uint64_t)md.query_heads * 128, kv = (uint64_t)md.kv_heads * 128,
                 in = md.intermediate, v = md.vocabulary;
  switch (kind) {
    case FH_LANGUAGE_MODEL_HEAD: *rows = v; *cols = h; return true;
    case FH_TOKEN_EMBEDDING: *rows = v; *cols = h; return true;
    case FH_FINAL_NORM: *rows = 1; *cols = h; return true;
    case FH_INPUT_LAYER_NORM: *rows = 1; *cols = h; return true;
    case FH_POST_ATTENTION_LAYER_NORM: *rows = 1; *cols = h; return true;
    case FH_QUERY_NORM: *rows = 1; *cols = 128; return true;
    case FH_KEY_NORM: *rows = 1; *cols = 128; return true;
    case FH_QUERY_PROJECTION: *rows = q; *cols = h; return true;
    case FH_KEY_PROJECTION: *rows = kv; *cols = h; return true;
    case FH_VALUE_PROJECTION: *rows = kv; *cols = h; return true;
    case FH_OUTPUT_PROJECTION: *rows = h; *cols = q; return true;
    case FH_GATE_PROJECTION: *rows = in; *cols = h; return true;
    case FH_UP_PROJECTION: *rows = in; *cols = h; return true;
    case FH_DOWN_PROJECTION: *rows = h; *cols = in; return true;
    default: return false;
  }
}

template <typename T>
fh_status dalloc(fh_ctx* ctx, T** out, uint64_t count) {
  void* p = nullptr;
  uint64_t bytes = std::max<uint64_t>(count * sizeof(T), 256);
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) return fail(ctx, FH_ERR_OUT_OF_MEMORY, "hipMalloc of " + std::to_string(bytes) + " bytes failed");
  ctx->device_allocs.push_back(p);
  *out = reinterpret_cast<T*>(p);
  return FH_OK;
}

template <typename T>
fh_status halloc(fh_ctx* ctx, T** out, uint64_t count, unsigned flags = hipHostMallocDefault) {
  void* p = nullptr;
  hipError_t e = hipHostMalloc(&p, std::max<uint64_t>(count * sizeof(T), 64), flags);
  if (e != hipSuccess) return fail(ctx, FH_ERR_OUT_OF_MEMORY, "hipHostMalloc failed");
  ctx->host_allocs.push_back(p);
  *out = reinterpret_cast<T*>(p);
  return FH_OK;
}

bool all_weights_present(const fh_ctx* ctx) {
  for (uint32_t k = 0; k <= FH_FINAL_NORM; ++k) {
    if (k == FH_LANGUAGE_MODEL_HEAD && ctx->md.tied_embedding) continue;
    if (!ctx->have[k]) return false;
  }
  for (uint32_t l = 0; l < ctx->md.layers; ++l)
    for (uint32_t k = FH_INPUT_LAYER_NORM; k <= FH_DOWN_PROJECTION; ++k)
      if (!ctx->have[tensor_index(k, l, ctx->md.layers)]) return false;
  return true;
}

uint16_t* kv_cache(fh_ctx* ctx, uint32_t layer, uint32_t which) {
  return ctx->kv + ((uint64_t)layer * 2 + which) * ctx->kv_slab_elems;
}

// Places a row-major tensor held in ctx->staging into its resident slot.
fh_status place_from_staging(fh_ctx* ctx, uint32_t kind, uint32_t layer) {
  uint64_t rows = 0, cols = 0;
  tensor_shape(ctx->md, kind, &rows, &cols);
  hipStream_t s = ctx->stream;
  const uint32_t q = ctx->md.query_heads * 128, kvc = ctx->md.kv_heads * 128;
  hipError_t e = hipSuccess;
  if (is_global(kind)) {
    if (kind == FH_FINAL_NORM)
      e = hipMemcpyAsync(ctx->final_norm, ctx->staging, cols * 2, hipMemcpyDeviceToDevice, s);
    else
      e = fh::launch_tile_weight(ctx->staging, kind == FH_TOKEN_EMBEDDING ? ctx->embed : ctx->head, (uint32_t)rows,
                                 (uint32_t)cols, 1, 0, s);
  } else {
    LayerWeights& L = ctx->layers[layer];
    const uint32_t H = ctx->md.hidden;
    switch (kind) {
      case FH_INPUT_LAYER_NORM: e = hipMemcpyAsync(L.in_norm, ctx->staging, cols * 2, hipMemcpyDeviceToDevice, s); break;
      case FH_POST_ATTENTION_LAYER_NORM: e = hipMemcpyAsync(L.post_norm, ctx->staging, cols * 2, hipMemcpyDeviceToDevice, s); break;
      case FH_QUERY_NORM: e = hipMemcpyAsync(L.q_norm, ctx->staging, cols * 2, hipMemcpyDeviceToDevice, s); break;
      case FH_KEY_NORM: e = hipMemcpyAsync(L.k_norm, ctx->staging, cols * 2, hipMemcpyDeviceToDevice, s); break;
      case FH_QUERY_PROJECTION: e = fh::launch_tile_weight(ctx->staging, L.qkv, q, H, 1, 0, s); break;
      case FH_KEY_PROJECTION: e = fh::launch_tile_weight(ctx->staging, L.qkv + (uint64_t)q * H, kvc, H, 1, 0, s); break;
      case FH_VALUE_PROJECTION: e = fh::launch_tile_weight(ctx->staging, L.qkv + (uint64_t)(q + kvc) * H, kvc, H, 1, 0, s); break;
      case FH_OUTPUT_PROJECTION: e = fh::launch_tile_weight(ctx->staging, L.o, H, q, 1, 0, s); break;
      case FH_GATE_PROJECTION: e = fh::launch_tile_weight(ctx->staging, L.gu, ctx->md.intermediate, H, 2, 0, s); break;
      case FH_UP_PROJECTION: e = fh::launch_tile_weight(ctx->staging, L.gu, ctx->md.intermediate, H, 2, 1, s); break;
      case FH_DOWN_PROJECTION: e = fh::launch_tile_weight(ctx->staging, L.down, H, ctx->md.intermediate, 1, 0, s); break;
      default: return fail(ctx, FH_ERR_INVALID_ARGUMENT, "unknown tensor kind");
    }
  }
  if (e != hipSuccess) return hip_fail(ctx, e, "placing weight");
  // The staging buffer is reused by the next upload: finish this one first.
  FH_HIP(ctx, hipStreamSynchronize(s));
  ctx->have[tensor_index(kind, layer, ctx->md.layers)] = 1;
  return FH_OK;
}

fh_status check_kind_layer(fh_ctx* ctx, uint32_t kind, uint32_t layer) {
  if (kind > FH_DOWN_PROJECTION) return fail(ctx, FH_ERR_INVALID_ARGUMENT, "tensor kind out of range");
  if (!is_global(kind) && layer >= ctx->md.layers) return fail(ctx, FH_ERR_INVALID_ARGUMENT, "layer out of range");
  if (kind == FH_LANGUAGE_MODEL_HEAD && ctx->md.tied_embedding)
    return fail(ctx, FH_ERR_INVALID_ARGUMENT, "tied model: the LM head is the token embedding");
  return FH_OK;
}

// ---- batch validation (batched.rs:1678-1744, 1519-1530) -------------------
fh_status validate_batch(fh_ctx* ctx, uint64_t batch_id, const fh_row* rows, uint32_t nrows,
                         const uint32_t* output_rows, uint32_t nout) {
  if (ctx->poisoned)
    return fail(ctx, FH_ERR_POISONED, "batched execution is closed, poisoned, or missing its v8 head profile");
  if (!all_weights_present(ctx)) return fail(ctx, FH_ERR_STATE, "model weights are not resident");
  const uint32_t max_rows = std::max(ctx->opt.row_capacity, ctx->opt.prefill_rows);
  if (batch_id <= ctx->last_batch || nrows == 0 || nrows > max_rows || rows == nullptr)
    return fail(ctx, FH_ERR_INVALID_BATCH, "foreign, stale, or invalid prepared GPU batch");
  if (nrows > ctx->opt.row_capacity && nout > kMaxPrefillOutputs)
    return fail(ctx, FH_ERR_OUTPUT_ROWS, "output rows must be unique, ascending, and within the batch");
  const uint32_t P = ctx->opt.physical_pages, stride = ctx->opt.page_table_stride;
  const uint64_t gen = ++ctx->stamp;
  // Pass 1, one visit per listed page: page -> (sequence, logical) ownership
  // over every row's list, and whether a row lists a page twice (the page's
  // last listing row is this row already).
  std::vector<uint8_t>& dup = ctx->row_dup;
  dup.assign(nrows, 0);
  fh_ctx::PageOwner* owner = ctx->page_owner.data();
  for (uint32_t i = 0; i < nrows; ++i) {
    const fh_row& r = rows[i];
    if (r.page_count > stride || (r.page_count && r.pages == nullptr))
      return fail(ctx, FH_ERR_INVALID_ROW, "invalid paged row geometry or aliased write slot");
    uint8_t row_dup = 0;
    for (uint32_t j = 0; j < r.page_count; ++j) {
      const uint32_t pg = r.pages[j];
      if (pg >= P) return fail(ctx, FH_ERR_INVALID_ROW, "invalid paged row geometry or aliased write slot");
      fh_ctx::PageOwner& o = owner[pg];
      if (o.stamp != gen) {
        o.stamp = gen;
        o.sequence = r.sequence;
        o.logical = j;
        o.conflict = 0;
        o.multi = 0;
      } else {
        row_dup |= o.row == i;
        o.multi |= o.row != i;
        if (o.sequence != r.sequence || o.logical != j) o.conflict = 1;
      }
      o.row = i;
    }
    dup[i] = row_dup;
  }
  // Pass 2, per row in order: geometry, unique pages, unique write slots.
  std::vector<uint64_t>& slots = ctx->slot_scratch;
  slots.clear();
  for (uint32_t i = 0; i < nrows; ++i) {
    const fh_row& r = rows[i];
    const uint32_t logical = r.position / kPageTokens;
    if (r.position >= ctx->opt.context_tokens || r.token >= ctx->md.vocabulary || logical >= r.page_count ||
        r.pages[logical] != r.writable_page)
      return fail(ctx, FH_ERR_INVALID_ROW, "invalid paged row geometry or aliased write slot");
    if (dup[i]) return fail(ctx, FH_ERR_INVALID_ROW, "invalid paged row geometry or aliased write slot");
    slots.push_back((uint64_t)r.pages[logical] * kPageTokens + r.position % kPageTokens);
    const fh_ctx::PageOwner& o = owner[r.pages[logical]];
    if (o.conflict || o.sequence != r.sequence || o.logical != logical)
      return fail(ctx, FH_ERR_SHARED_PAGE, "batch writes a page shared with another sequence or logical position");
  }
  // A row may read another row's new slot only where that row's written
  // page is listed by another row (rows of one sequence in one batch); the
  // decode step then keeps the QK-norm/KV append as a launch of its own.
  ctx->batch_private_slots = true;
  for (uint32_t i = 0; i < nrows; ++i)
    if (owner[rows[i].writable_page].multi) ctx->batch_private_slots = false;
  std::sort(slots.begin(), slots.end());
  if (std::adjacent_find(slots.begin(), slots.end()) != slots.end())
    return fail(ctx, FH_ERR_INVALID_ROW, "invalid paged row geometry or aliased write slot");
  for (uint32_t i = 0; i < nout; ++i)
    if (output_rows[i] >= nrows || (i > 0 && output_rows[i] <= output_rows[i - 1]))
      return fail(ctx, FH_ERR_OUTPUT_ROWS, "output rows must be unique, ascending, and within the batch");
  return FH_OK;
}

// ---- the step ---------------------------------------------------------------
// Issues a step's launches in order, or, dry, only counts them: the dispatch
// preflight runs the same enqueue code as the step, so the two cannot drift.
struct Enq {
  fh_ctx* ctx;
  bool dry = false;
  uint32_t next_event = 0;
  uint64_t launches = 0;
  hipError_t first_error = hipSuccess;
  uint32_t first_error_class = 0;
  uint64_t first_error_launch = 0;

  template <typename F>
  void run(uint32_t cls, F&& f) {
    if (dry) {
      ++launches;
      return;
    }
    const bool prof = ctx->profiling;
    hipEvent_t b = nullptr, e = nullptr;
    if (prof && next_event + 1 < ctx->prof_events.size()) {
      b = ctx->prof_events[next_event++];
      e = ctx->prof_events[next_event++];
      hipEventRecord(b, ctx->stream);
    }
    hipError_t err = f();
    if (err != hipSuccess && first_error == hipSuccess) {
      first_error = err;
      first_error_class = cls;
      first_error_launch = launches;
    }
    ++launches;
    if (b) {
      hipEventRecord(e, ctx->stream);
      ctx->prof_launches.push_back({cls, b, e});
    }
  }
};

// Whether this decode batch runs the QK-norm/RoPE/KV append inside the
// attention partitions: every row's written page private to that row, a
// model shape the fused kernel covers, and a launch small enough to merge
// its partitions in the same launch (attn_fuse_merge). Each partition then
// forms its query heads itself, and the serial square sum of the norm (128
// dependent adds per head) sits before its scores. Measured on MI355X
// (alternating runs on one GPU, graph replays): one Qwen3-8B row at a
// 4096-token context 3.538 -> 3.467-3.483 ms per step; 32 rows of the 8B at
// contexts U[512, 8192] 4311 against 4252-4347 tok/s and 32 rows of the
// 0.6B at U[128, 2048] 17.5-17.6k against 16.8-17.3k tok/s, where the
// longer partitions cost more than the launch they save. Models with at
// most 2 query heads per KV head (Qwen3-0.6B) take it at any size once V is
// requested after the scores there (occupancy kept at 3 workgroups per CU):
// 32 rows 1.741-1.742 -> 1.733-1.734 ms device time per step.
bool step_runs_qkn(const fh_ctx* ctx, uint32_t rows) {
  const uint32_t split = fh::attn_split_pages(rows, ctx->md.query_heads, ctx->opt.context_tokens);
  return ctx->batch_private_slots &&
         fh::attention_qkn_supported(ctx->md.query_heads, ctx->md.kv_heads, ctx->s_qkv) &&
         (fh::attn_fuse_merge(rows, ctx->md.kv_heads, ctx->opt.context_tokens, split) ||
          ctx->md.query_heads <= 2 * ctx->md.kv_heads);
}

fh::AttnQkn step_qkn_args(fh_ctx* ctx, uint32_t l) {
  const LayerWeights& W = ctx->layers[l];
  return fh::AttnQkn{ctx->qkv_part,   ctx->s_qkv,     fh::kMaxRows,         W.q_norm,
                     W.k_norm,        ctx->cos_t,     ctx->sin_t,           kv_cache(ctx, l, 0),
                     kv_cache(ctx, l, 1), ctx->md.rms_epsilon};
}

// Enqueues (or, dry, only counts) the launches of a decode step of R rows.
hipError_t enqueue_step(fh_ctx* ctx, uint32_t R, uint64_t* launches, bool dry = false) {
  const fh_model_desc& md = ctx->md;
  const fh_ctx_options& op = ctx->opt;
  hipStream_t s = ctx->stream;
  const uint32_t H = md.hidden, QH = md.query_heads, KVH = md.kv_heads, Q = QH * 128, I = md.intermediate;
  const uint32_t cap = op.row_capacity, stride = op.page_table_stride, P = op.physical_pages,
                 C = op.context_tokens;
  const uint32_t* d_pos = ctx->d_meta + cap;
  const uint32_t* d_tab = ctx->d_meta + 2 * cap;
  uint32_t* err = ctx->err;
  Enq q{ctx, dry};
  if (!dry) (void)hipGetLastError();  // launch statuses below then belong to these launches
  uint64_t n = 0;
  auto L = [&](uint32_t cls, auto&& f) {
    q.run(cls, f);
    ++n;
  };
  // Residual stream: `hidden` (row-major bf16). Projection inputs (xn, attn,
  // act) are in activation tile order. The O and down projections leave
  // split-K FP32 partials that the next residual + RMSNorm folds into
  // `hidden` (one rounding, as the TP1 residual); the QKV partials are folded
  // by the QK-norm kernel.
  const uint32_t sq = ctx->s_qkv, so = ctx->s_o, sd = ctx->s_down;
  const uint32_t split = fh::attn_split_pages(R, QH, C);
  const bool fuse = fh::attn_fuse_merge(R, KVH, C, split);
  const bool qkn = step_runs_qkn(ctx, R);
  // The step's tokens, positions and page tables come in from the pinned
  // host mirror by the first launch, so a replayed graph needs no copy beside it.
  const uint32_t meta_words = 2 * cap + R * stride;
  L(FH_KC_EMBEDDING, [&] {
    return fh::launch_step_embed(ctx->h_meta, ctx->d_meta, meta_words, ctx->embed, ctx->hidden, R, H, md.vocabulary,
                                 err, s);
  });
  // One row: each residual + RMSNorm runs in the prologue of the projection
  // that consumes the normalized row (QKV, gate/up, LM head), so a layer is 5
  // launches. Every workgroup of that projection reads the residual row and
  // the split-K slabs; one writes the folded row to the residual stream's
  // other buffer (`cur` alternates between hidden and hidden_alt), so no
  // workgroup reads a row another one is writing.
  const bool row_norm = R == 1 && ctx->row_norm_fused;
  uint16_t* cur = ctx->hidden;
  auto fold_into = [&](uint32_t slabs) {
    return slabs == 0 ? cur : cur == ctx->hidden ? ctx->hidden_alt : ctx->hidden;
  };
  auto capture_copy = [&](uint32_t layer) {
    L(FH_KC_RMSNORM, [&] {
      return fh::launch_copy_u16(cur, ctx->capture + (uint64_t)layer * ctx->capture_rows * H, (uint64_t)R * H, s);
    });
  };
  for (uint32_t l = 0; l < md.layers; ++l) {
    const LayerWeights& W = ctx->layers[l];
    uint16_t* kc = kv_cache(ctx, l, 0);
    uint16_t* vc = kv_cache(ctx, l, 1);
    const uint32_t fold = l == 0 ? 0 : sd;
    if (row_norm) {
      uint16_t* next = fold_into(fold);
      const fh::RowNormArgs na{cur, next, ctx->down_part, fold, fh::partial_slab_rows(1), W.in_norm, md.rms_epsilon};
      L(FH_KC_QKV_GEMM, [&] {
        return fh::launch_gemm_rownorm(W.qkv, ctx->nqkv, H, FH_EPI_PARTIAL, sq, na, ctx->qkv_part, ctx->nqkv, err, s);
      });
      cur = next;
      if (ctx->capture && l > 0) capture_copy(l - 1);
    } else {
      L(FH_KC_RMSNORM, [&] {
        return fh::launch_residual_rmsnorm(ctx->hidden, ctx->down_part, fold, W.in_norm, ctx->xn, 1, R, H,
                                           md.rms_epsilon, err, s);
      });
      if (ctx->capture && l > 0) capture_copy(l - 1);
      L(FH_KC_QKV_GEMM, [&] {
        return fh::launch_gemm(ctx->xn, W.qkv, R, ctx->nqkv, H, FH_EPI_PARTIAL, sq, nullptr, ctx->qkv_part,
                               ctx->nqkv, err, s);
      });
    }
    // Where no row reads another row's new slot, the attention partitions
    // run the QK-norm/RoPE/KV append themselves (same arithmetic, bit for
    // bit), which saves a launch per layer.
    if (!qkn)
      L(FH_KC_QKNORM_ROPE_KV, [&] {
        return fh::launch_qknorm_rope_kv(nullptr, ctx->qkv_part, sq, W.q_norm, W.k_norm, ctx->cos_t, ctx->sin_t,
                                         d_pos, d_tab, ctx->qrot, kc, vc, R, QH, KVH, stride, P, C, md.rms_epsilon,
                                         err, s);
      });
    const fh::AttnQkn qa = step_qkn_args(ctx, l);
    L(FH_KC_ATTENTION, [&] {
      return fh::launch_attention_partial(ctx->qrot, kc, vc, d_pos, d_tab, ctx->attn_part, ctx->attn, 1, 0, R, R, QH,
                                          KVH, stride, P, C, split, fuse ? ctx->attn_count : nullptr, err, s,
                                          qkn ? &qa : nullptr);
    });
    if (!fuse)
      L(FH_KC_ATTENTION_MERGE, [&] {
        return fh::launch_attention_merge(ctx->attn_part, d_pos, ctx->attn, 1, 0, R, R, QH, C, split, err, s);
      });
    L(FH_KC_O_GEMM, [&] {
      return fh::launch_gemm(ctx->attn, W.o, R, H, Q, FH_EPI_PARTIAL, so, nullptr, ctx->o_part, H, err, s);
    });
    if (row_norm) {
      uint16_t* next = fold_into(so);
      const fh::RowNormArgs na{cur, next, ctx->o_part, so, fh::partial_slab_rows(1), W.post_norm, md.rms_epsilon};
      L(FH_KC_GATE_UP_GEMM, [&] {
        return fh::launch_gemm_rownorm(W.gu, 2 * I, H, FH_EPI_SWIGLU, 1, na, ctx->act, I, err, s);
      });
      cur = next;
    } else {
      L(FH_KC_RMSNORM, [&] {
        return fh::launch_residual_rmsnorm(ctx->hidden, ctx->o_part, so, W.post_norm, ctx->xn, 1, R, H,
                                           md.rms_epsilon, err, s);
      });
      L(FH_KC_GATE_UP_GEMM, [&] {
        return fh::launch_gemm(ctx->xn, W.gu, R, 2 * I, H, FH_EPI_SWIGLU, 1, nullptr, ctx->act, I, err, s);
      });
    }
    L(FH_KC_DOWN_GEMM, [&] {
      return fh::launch_gemm(ctx->act, W.down, R, H, I, FH_EPI_PARTIAL, sd, nullptr, ctx->down_part, H, err, s);
    });
  }
  if (row_norm) {
    uint16_t* next = fold_into(sd);
    const fh::RowNormArgs na{cur, next, ctx->down_part, sd, fh::partial_slab_rows(1), ctx->final_norm, md.rms_epsilon};
    L(FH_KC_HEAD_GEMM, [&] {
      return fh::launch_gemm_rownorm(ctx->head, md.vocabulary, H, FH_EPI_F32, 1, na, ctx->logits, md.vocabulary, err,
                                     s);
    });
    cur = next;
    if (ctx->capture) capture_copy(md.layers - 1);
  } else {
    L(FH_KC_RMSNORM, [&] {
      return fh::launch_residual_rmsnorm(ctx->hidden, ctx->down_part, sd, ctx->final_norm, ctx->xn, 1, R, H,
                                         md.rms_epsilon, err, s);
    });
    if (ctx->capture) capture_copy(md.layers - 1);
    L(FH_KC_HEAD_GEMM, [&] {
      return fh::launch_gemm(ctx->xn, ctx->head, R, md.vocabulary, H, FH_EPI_F32, 1, nullptr, ctx->logits,
                             md.vocabulary, err, s);
    });
  }
  L(FH_KC_ARGMAX, [&] {
    return fh::launch_argmax(ctx->logits, R, md.vocabulary, ctx->argmax_scratch, ctx->choices, err, s, ctx->h_out,
                             ctx->h_out + cap, ctx->h_out + cap + 1);
  });
  ++n;  // argmax is two launches
  *launches = n;
  if (dry) return hipSuccess;
  if (q.first_error != hipSuccess)
    ctx->launch_detail = std::string(" (kernel class ") + std::to_string(q.first_error_class) + ", launch " +
                         std::to_string(q.first_error_launch) + ")";
  return q.first_error;
}

void collect_profile(fh_ctx* ctx) {
  for (uint32_t c = 0; c < FH_KC_COUNT; ++c) {
    ctx->class_ms[c] = 0.f;
    ctx->class_launches[c] = 0;
  }
  for (const auto& pl : ctx->prof_launches) {
    float ms = 0.f;
    hipEventElapsedTime(&ms, pl.begin, pl.end);
    ctx->class_ms[pl.cls] += ms;
    ctx->class_launches[pl.cls] += 1;
  }
}

std::string error_bits(uint32_t e) {
  std::string s;
  if (e & fh::ERR_NONFINITE) s += " nonfinite-value";
  if (e & fh::ERR_TOKEN) s += " token-out-of-vocabulary";
  if (e & fh::ERR_POSITION) s += " position-out-of-context";
  if (e & fh::ERR_PAGE) s += " page-out-of-pool";
  return s;
}

}  // namespace

namespace fh {
// Message for fh_last_error(NULL) after a failed context-free call.
void set_thread_error(const char* msg) { g_create_error = msg; }
}  // namespace fh

extern "C" {

const char* fh_last_error(const fh_ctx* ctx) { return ctx ? ctx->error.c_str() : g_create_error.c_str(); }

fh_status fh_create(const fh_model_desc* md_in, const fh_ctx_options* op_in, fh_ctx** out) {
  if (!md_in || !op_in || !out) return fail(nullptr, FH_ERR_INVALID_ARGUMENT, "null argument");
  *out = nullptr;
  const fh_model_desc md = *md_in;
  const fh_ctx_options op = *op_in;
  if (md.layers == 0 || md.head_dim != 128 || md.kv_heads == 0 || md.query_heads % md.kv_heads != 0 ||
      (md.query_heads / md.kv_heads) > 8 || ((md.query_heads / md.kv_heads) & ((md.query_heads / md.kv_heads) - 1)) ||
      md.hidden % 256 != 0 || md.hidden > 8192 || md.intermediate % 256 != 0 || md.vocabulary % 16 != 0 ||
      md.vocabulary == 0 || (md.query_heads * 128) % 256 != 0 || md.query_heads + md.kv_heads > 64)
    return fail(nullptr, FH_ERR_INVALID_ARGUMENT, "unsupported model shape");
  if (op.row_capacity == 0 || op.row_capacity > kMaxRows || op.physical_pages == 0 || op.context_tokens == 0 ||
      op.page_table_stride == 0 || op.page_table_stride * kPageTokens < op.context_tokens ||
      (op.prefill_rows != 0 && (op.prefill_rows <= op.row_capacity || op.prefill_rows > 16384)))
    return fail(nullptr, FH_ERR_INVALID_ARGUMENT, "unsupported context options");
  if (op.prefill_rows && md.vocabulary % 128 != 0)
    return fail(nullptr, FH_ERR_INVALID_ARGUMENT, "unsupported model shape for prefill (vocabulary % 128)");

  fh_ctx* ctx = new fh_ctx();
  ctx->md = md;
  ctx->opt = op;
  auto bail = [&](fh_status st) {
    g_create_error = ctx->error;
    fh_destroy(ctx);
    return st;
  };
  hipError_t e = hipSetDevice(op.device);
  if (e != hipSuccess) return bail(hip_fail(ctx, e, "hipSetDevice"));
  e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) return bail(hip_fail(ctx, e, "hipStreamCreate"));
  if ((e = hipEventCreate(&ctx->ev_begin)) != hipSuccess || (e = hipEventCreate(&ctx->ev_end)) != hipSuccess)
    return bail(hip_fail(ctx, e, "hipEventCreate"));

  const uint32_t H = md.hidden, Q = md.query_heads * 128, KV = md.kv_heads * 128, I = md.intermediate,
                 V = md.vocabulary, cap = op.row_capacity;
  ctx->nqkv = Q + 2 * KV;
  ctx->layers.resize(md.layers);
  ctx->have.assign(3 + 11 * md.layers, 0);
  fh_status st;
#define TRY(x)                  \
  if ((st = (x)) != FH_OK) {    \
    return bail(st);            \
  }
  TRY(dalloc(ctx, &ctx->embed, (uint64_t)V * H));
  if (md.tied_embedding)
    ctx->head = ctx->embed;
  else
    TRY(dalloc(ctx, &ctx->head, (uint64_t)V * H));
  TRY(dalloc(ctx, &ctx->final_norm, H));
  for (auto& L : ctx->layers) {
    TRY(dalloc(ctx, &L.qkv, (uint64_t)ctx->nqkv * H));
    TRY(dalloc(ctx, &L.o, (uint64_t)H * Q));
    TRY(dalloc(ctx, &L.gu, (uint64_t)2 * I * H));
    TRY(dalloc(ctx, &L.down, (uint64_t)H * I));
    TRY(dalloc(ctx, &L.in_norm, H));
    TRY(dalloc(ctx, &L.post_norm, H));
    TRY(dalloc(ctx, &L.q_norm, 128));
    TRY(dalloc(ctx, &L.k_norm, 128));
  }
  ctx->staging_elems = std::max<uint64_t>({(uint64_t)V * H, (uint64_t)I * H, (uint64_t)Q * H});
  TRY(dalloc(ctx, &ctx->staging, ctx->staging_elems));
  ctx->kv_slab_elems = (uint64_t)op.physical_pages * kPageTokens * KV;
  TRY(dalloc(ctx, &ctx->kv, ctx->kv_slab_elems * 2 * md.layers));
  TRY(dalloc(ctx, &ctx->cos_t, (uint64_t)op.context_tokens * 64));
  TRY(dalloc(ctx, &ctx->sin_t, (uint64_t)op.context_tokens * 64));
  TRY(dalloc(ctx, &ctx->hidden, (uint64_t)cap * H));
  // Activation-tile buffers always hold 32 rows (two 16-row m-tiles).
  TRY(dalloc(ctx, &ctx->xn, (uint64_t)kMaxRows * H));
  TRY(dalloc(ctx, &ctx->qrot, (uint64_t)cap * Q));
  TRY(dalloc(ctx, &ctx->attn, (uint64_t)kMaxRows * Q));
  TRY(dalloc(ctx, &ctx->act, (uint64_t)kMaxRows * I));
  ctx->s_qkv = fh::gemm_default_splits(ctx->nqkv, H);
  ctx->s_o = fh::gemm_default_splits(H, Q);
  ctx->s_down = fh::gemm_default_splits(H, I);
  // One-row steps fold and normalize the row inside the QKV, gate/up and LM
  // head projections where the fused launch covers all of their shapes.
  ctx->row_norm_fused = fh::gemm_rownorm_supported(ctx->nqkv, H, FH_EPI_PARTIAL, ctx->s_qkv, 0) &&
                        fh::gemm_rownorm_supported(ctx->nqkv, H, FH_EPI_PARTIAL, ctx->s_qkv, ctx->s_down) &&
                        fh::gemm_rownorm_supported(2 * I, H, FH_EPI_SWIGLU, 1, ctx->s_o) &&
                        fh::gemm_rownorm_supported(V, H, FH_EPI_F32, 1, ctx->s_down);
  if (ctx->row_norm_fused) TRY(dalloc(ctx, &ctx->hidden_alt, H));
  TRY(dalloc(ctx, &ctx->qkv_part, (uint64_t)ctx->s_qkv * kMaxRows * ctx->nqkv));
  TRY(dalloc(ctx, &ctx->o_part, (uint64_t)ctx->s_o * kMaxRows * H));
  TRY(dalloc(ctx, &ctx->down_part, (uint64_t)ctx->s_down * kMaxRows * H));
  TRY(dalloc(ctx, &ctx->logits, (uint64_t)cap * V));
  TRY(dalloc(ctx, &ctx->attn_part, (uint64_t)cap * md.query_heads *
                                        fh::attn_max_splits(op.context_tokens, fh::kAttnMinSplitPages) *
                                        fh::kAttnPartialFloats));
  TRY(dalloc(ctx, &ctx->attn_count, (uint64_t)cap * md.kv_heads));
  TRY(dalloc(ctx, reinterpret_cast<uint8_t**>(&ctx->argmax_scratch), fh_argmax_scratch_bytes(cap)));
  TRY(dalloc(ctx, &ctx->choices, cap));
  TRY(dalloc(ctx, &ctx->err, 64));
  ctx->capture_rows = std::max(cap, op.prefill_rows);
  if (op.capture_hidden) TRY(dalloc(ctx, &ctx->capture, (uint64_t)md.layers * ctx->capture_rows * H));
  const uint64_t meta = 2ull * cap + (uint64_t)cap * op.page_table_stride;
  TRY(dalloc(ctx, &ctx->d_meta, meta));
  // Decode steps read their metadata from, and publish their choices into,
  // these two buffers from inside the step's kernels: coherent pinned memory.
  TRY(halloc(ctx, &ctx->h_meta, meta, hipHostMallocCoherent));
  TRY(halloc(ctx, &ctx->h_out, 2 * cap + 1, hipHostMallocCoherent));
  if (op.prefill_rows) {
    auto& p = ctx->pre;
    const uint32_t P = op.prefill_rows;
    const uint64_t tiled_rows = (uint64_t)fh::act_mtiles(P) * 16;
    const uint64_t out_tiled_rows = (uint64_t)fh::act_mtiles(kMaxPrefillOutputs) * 16;
    TRY(dalloc(ctx, &p.hidden, (uint64_t)P * H));
    TRY(dalloc(ctx, &p.xn, tiled_rows * H));
    TRY(dalloc(ctx, &p.qkv, (uint64_t)P * ctx->nqkv));
    TRY(dalloc(ctx, &p.qrot, (uint64_t)P * Q));
    TRY(dalloc(ctx, &p.attn, tiled_rows * Q));
    TRY(dalloc(ctx, &p.act, tiled_rows * I));
    TRY(dalloc(ctx, &p.out_hidden, (uint64_t)kMaxPrefillOutputs * H));
    TRY(dalloc(ctx, &p.out_xn, out_tiled_rows * H));
    p.s_qkv = fh::gemm_panel_splits(ctx->nqkv, H);
    p.s_o = fh::gemm_panel_splits(H, Q);
    p.s_down = fh::gemm_panel_splits(H, I);
    const uint64_t part_floats =
        std::max({(uint64_t)p.s_qkv * fh::kPanelRows * ctx->nqkv, (uint64_t)p.s_o * fh::kPanelRows * H,
                  (uint64_t)p.s_down * fh::kPanelRows * H, (uint64_t)ctx->s_qkv * kMaxRows * ctx->nqkv,
                  (uint64_t)ctx->s_o * kMaxRows * H, (uint64_t)ctx->s_down * kMaxRows * H});
    TRY(dalloc(ctx, &p.part, part_floats));
    TRY(dalloc(ctx, &p.logits, (uint64_t)kMaxPrefillOutputs * V));
    TRY(dalloc(ctx, reinterpret_cast<uint8_t**>(&p.argmax_scratch), fh_argmax_scratch_bytes(kMaxPrefillOutputs)));
    TRY(dalloc(ctx, &p.choices, kMaxPrefillOutputs));
    const uint64_t pmeta = 3ull * P + kMaxPrefillOutputs + (uint64_t)P * op.page_table_stride;
    TRY(dalloc(ctx, &p.d_meta, pmeta));
    TRY(halloc(ctx, &p.h_meta, pmeta));
    TRY(halloc(ctx, &p.h_out, kMaxPrefillOutputs + 1));
    // Padding rows of the tiled buffers are read (never used) by the GEMM.
    e = fh::launch_fill_u16(p.xn, tiled_rows * H, 0, ctx->stream);
    if (e == hipSuccess) e = fh::launch_fill_u16(p.attn, tiled_rows * Q, 0, ctx->stream);
    if (e == hipSuccess) e = fh::launch_fill_u16(p.act, tiled_rows * I, 0, ctx->stream);
    if (e == hipSuccess) e = fh::launch_fill_u16(p.out_xn, out_tiled_rows * H, 0, ctx->stream);
    if (e != hipSuccess) return bail(hip_fail(ctx, e, "initialising prefill buffers"));
  }

  // RoPE table exactly as rope_bytes (tp_execution.rs:1440-1450): f64
  // theta^(-pair/64), angle = position * inverse_frequency, cos/sin in f64,
  // narrowed to f32.
  {
    std::vector<float> c((uint64_t)op.context_tokens * 64), sn((uint64_t)op.context_tokens * 64);
    for (uint32_t p = 0; p < op.context_tokens; ++p)
      for (uint32_t i = 0; i < 64; ++i) {
        const double inv = std::pow((double)md.rope_theta, -(double)i / 64.0);
        const double angle = (double)p * inv;
        c[(uint64_t)p * 64 + i] = (float)std::cos(angle);
        sn[(uint64_t)p * 64 + i] = (float)std::sin(angle);
      }
    e = hipMemcpy(ctx->cos_t, c.data(), c.size() * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(ctx->sin_t, sn.data(), sn.size() * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) return bail(hip_fail(ctx, e, "uploading the RoPE table"));
  }
  // Deterministic contents for never-written KV slots and activations.
  e = fh::launch_fill_u16(ctx->kv, ctx->kv_slab_elems * 2 * md.layers, 0, ctx->stream);
  if (e == hipSuccess) e = fh::launch_fill_u16(ctx->hidden, (uint64_t)cap * H, 0, ctx->stream);
  if (e == hipSuccess) e = fh::launch_fill_u16(reinterpret_cast<uint16_t*>(ctx->attn_count), 2ull * cap * md.kv_heads, 0,
                                               ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return bail(hip_fail(ctx, e, "initialising the KV pool"));

  ctx->page_owner.assign(op.physical_pages, fh_ctx::PageOwner{});
#undef TRY
  *out = ctx;
  return FH_OK;
}

void fh_destroy(fh_ctx* ctx) {
  if (!ctx) return;
  if (ctx->stream) hipStreamSynchronize(ctx->stream);
  for (auto& kv : ctx->graphs) hipGraphExecDestroy(kv.second.exec);
  for (auto g : ctx->graph_defs) hipGraphDestroy(g);
  for (auto ev : ctx->prof_events) hipEventDestroy(ev);
  if (ctx->ev_begin) hipEventDestroy(ctx->ev_begin);
  if (ctx->ev_end) hipEventDestroy(ctx->ev_end);
  for (void* p : ctx->device_allocs) hipFree(p);
  for (void* p : ctx->host_allocs) hipHostFree(p);
  if (ctx->stream) hipStreamDestroy(ctx->stream);
  delete ctx;
}

fh_status fh_upload_weight(fh_ctx* ctx, uint32_t kind, uint32_t layer, const uint16_t* host, uint64_t elements) {
  if (!ctx || !host) return fail(ctx, FH_ERR_INVALID_ARGUMENT, "null argument");
  fh_status st = check_kind_layer(ctx, kind, layer);
  if (st != FH_OK) return st;
  uint64_t rows = 0, cols = 0;
  tensor_shape(ctx->md, kind, &rows, &cols);
  if (elements != rows * cols)
    return fail(ctx, FH_ERR_INVALID_ARGUMENT, "weight element count does not match the model shape");
  FH_HIP(ctx, hipMemcpy(ctx->staging, host, elements * 2, hipMemcpyHostToDevice));
  return place_from_staging(ctx, kind, layer);
}

fh_status fh_synthesize_weights(fh_ctx* ctx, uint64_t seed, float sigma) {
  if (!ctx) return FH_ERR_INVALID_ARGUMENT;
  const float scale = fh_synth_scale(sigma);
  auto one = [&](uint32_t kind, uint32_t layer) -> fh_status {
    uint64_t rows = 0, cols = 0;
    tensor_shape(ctx->md, kind, &rows, &cols);
    hipError_t e;
    if (rows == 1)
      e = fh::launch_fill_u16(ctx->staging, cols, 0x3f80, ctx->stream);  // norms = 1.0
    else
      e = fh::launch_synth_fill(ctx->staging, rows * cols, fh_synth_tensor_seed(seed, kind, layer), scale,
                                ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "synthesising a weight");
    return place_from_staging(ctx, kind, layer);
  };
  fh_status st;
  for (uint32_t k = 0; k <= FH_FINAL_NORM; ++k) {
    if (k == FH_LANGUAGE_MODEL_HEAD && ctx->md.tied_embedding) continue;
    if ((st = one(k, kNoLayer)) != FH_OK) return st;
  }
  for (uint32_t l = 0; l < ctx->md.layers; ++l)
    for (uint32_t k = FH_INPUT_LAYER_NORM; k <= FH_DOWN_PROJECTION; ++k)
      if ((st = one(k, l)) != FH_OK) return st;
  return FH_OK;
}

fh_status fh_download_weight(fh_ctx* ctx, uint32_t kind, uint32_t layer, uint16_t* host, uint64_t elements) {
  if (!ctx || !host) return fail(ctx, FH_ERR_INVALID_ARGUMENT, "null argument");
  fh_status st = check_kind_layer(ctx, kind, layer);
  if (st != FH_OK) return st;
  uint64_t rows = 0, cols = 0;
  tensor_shape(ctx->md, kind, &rows, &cols);
  if (elements != rows * cols) return fail(ctx, FH_ERR_INVALID_ARGUMENT, "element count mismatch");
  if (!ctx->have[tensor_index(kind, layer, ctx->md.layers)]) return fail(ctx, FH_ERR_STATE, "weight not resident");
  const uint32_t H = ctx->md.hidden, q = ctx->md.query_heads * 128, kvc = ctx->md.kv_heads * 128;
  const uint16_t* src = nullptr;
  bool tiled = true;
  if (is_global(kind)) {
    if (kind == FH_FINAL_NORM) {
      src = ctx->final_norm;
      tiled = false;
    } else {
      src = kind == FH_TOKEN_EMBEDDING ? ctx->embed : ctx->head;
    }
  } else {
    const LayerWeights& L = ctx->layers[layer];
    switch (kind) {
      case FH_INPUT_LAYER_NORM: src = L.in_norm; tiled = false; break;
      case FH_POST_ATTENTION_LAYER_NORM: src = L.post_norm; tiled = false; break;
      case FH_QUERY_NORM: src = L.q_norm; tiled = false; break;
      case FH_KEY_NORM: src = L.k_norm; tiled = false; break;
      case FH_QUERY_PROJECTION: src = L.qkv; break;
      case FH_KEY_PROJECTION: src = L.qkv + (uint64_t)q * H; break;
      case FH_VALUE_PROJECTION: src = L.qkv + (uint64_t)(q + kvc) * H; break;
      case FH_OUTPUT_PROJECTION: src = L.o; break;
      case FH_DOWN_PROJECTION: src = L.down; break;
      case FH_GATE_PROJECTION:
      case FH_UP_PROJECTION: {
        // Gather the even (gate) or odd (up) tiles back into row-major order.
        const uint32_t I = ctx->md.intermediate, kb = H / 32;
        std::vector<uint16_t> all((uint64_t)2 * I * H);
        FH_HIP(ctx, hipMemcpy(all.data(), L.gu, all.size() * 2, hipMemcpyDeviceToHost));
        const uint32_t parity = kind == FH_UP_PROJECTION ? 1 : 0;
        for (uint64_t n = 0; n < I; ++n)
          for (uint32_t k = 0; k < H; ++k) {
            const uint64_t tile_n = ((n >> 4) * 2 + parity) * 16 + (n & 15);
            host[n * H + k] = all[fh::tiled_offset((uint32_t)tile_n, k, H)];
          }
        (void)kb;
        return FH_OK;
      }
      default: return fail(ctx, FH_ERR_INVALID_ARGUMENT, "unknown tensor kind");
    }
  }
  if (tiled) {
    hipError_t e = fh::launch_untile_weight(src, ctx->staging, (uint32_t)rows, (uint32_t)cols, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "untile");
    FH_HIP(ctx, hipStreamSynchronize(ctx->stream));
    src = ctx->staging;
  }
  FH_HIP(ctx, hipMemcpy(host, src, elements * 2, hipMemcpyDeviceToHost));
  return FH_OK;
}

fh_status fh_kv_fill_synthetic(fh_ctx* ctx, uint64_t seed, float sigma, const fh_row* rows,
                               const uint64_t* keys, uint32_t nrows, uint32_t context_stride) {
  if (!ctx || !rows || !keys || nrows == 0) return fail(ctx, FH_ERR_INVALID_ARGUMENT, "null argument");
  const uint32_t stride = ctx->opt.page_table_stride;
  std::vector<uint32_t> table((uint64_t)nrows * stride, 0xffffffffu), lengths(nrows);
  uint32_t max_len = 0;
  for (uint32_t i = 0; i < nrows; ++i) {
    const fh_row& r = rows[i];
    const uint32_t need = (r.position + kPageTokens - 1) / kPageTokens;
    if (r.position > ctx->opt.context_tokens || r.position > context_stride || need > r.page_count ||
        r.page_count > stride)
      return fail(ctx, FH_ERR_INVALID_ROW, "KV prefix does not fit the row's pages");
    for (uint32_t j = 0; j < r.page_count; ++j) {
      if (r.pages[j] >= ctx->opt.physical_pages) return fail(ctx, FH_ERR_INVALID_ROW, "page outside the pool");
      table[(uint64_t)i * stride + j] = r.pages[j];
    }
    lengths[i] = r.position;
    max_len = std::max(max_len, r.position);
  }
  uint32_t *d_table = nullptr, *d_len = nullptr;
  uint64_t* d_keys = nullptr;
  FH_HIP(ctx, hipMalloc(&d_table, table.size() * 4));
  FH_HIP(ctx, hipMalloc(&d_len, nrows * 4));
  FH_HIP(ctx, hipMalloc(&d_keys, nrows * 8));
  hipError_t e = hipMemcpy(d_table, table.data(), table.size() * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(d_len, lengths.data(), nrows * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(d_keys, keys, nrows * 8, hipMemcpyHostToDevice);
  const float scale = fh_synth_scale(sigma);
  for (uint32_t l = 0; l < ctx->md.layers && e == hipSuccess && max_len > 0; ++l)
    for (uint32_t w = 0; w < 2 && e == hipSuccess; ++w)
      e = fh::launch_kv_fill(kv_cache(ctx, l, w), d_table, d_len, d_keys, nrows, stride, ctx->md.kv_heads,
                             fh_synth_tensor_seed(seed, FH_SYNTH_KIND_KV_KEY + w, l), scale, context_stride, max_len,
                             ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  hipFree(d_table);
  hipFree(d_len);
  hipFree(d_keys);
  if (e != hipSuccess) return hip_fail(ctx, e, "KV fill");
  return FH_OK;
}

fh_status fh_read_kv_page(fh_ctx* ctx, uint32_t layer, uint32_t which, uint32_t page, uint16_t* out,
                          uint64_t elements) {
  if (!ctx || !out || layer >= ctx->md.layers || which > 1 || page >= ctx->opt.physical_pages ||
      elements != (uint64_t)kPageTokens * ctx->md.kv_heads * 128)
    return fail(ctx, FH_ERR_INVALID_ARGUMENT, "bad KV page request");
  FH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  FH_HIP(ctx, hipMemcpy(out, kv_cache(ctx, layer, which) + (uint64_t)page * elements, elements * 2,
                        hipMemcpyDeviceToHost));
  return FH_OK;
}

fh_status fh_read_kv_cache(fh_ctx* ctx, uint32_t layer, uint32_t which, uint16_t* out, uint64_t elements) {
  if (!ctx || !out || layer >= ctx->md.layers || which > 1 || elements != ctx->kv_slab_elems)
    return fail(ctx, FH_ERR_INVALID_ARGUMENT, "bad KV cache request");
  FH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  FH_HIP(ctx, hipMemcpy(out, kv_cache(ctx, layer, which), elements * 2, hipMemcpyDeviceToHost));
  return FH_OK;
}

fh_status fh_write_kv_page(fh_ctx* ctx, uint32_t layer, uint32_t which, uint32_t page, const uint16_t* data,
                           uint64_t elements) {
  if (!ctx || !data || layer >= ctx->md.layers || which > 1 || page >= ctx->opt.physical_pages ||
      elements != (uint64_t)kPageTokens * ctx->md.kv_heads * 128)
    return fail(ctx, FH_ERR_INVALID_ARGUMENT, "bad KV page request");
  FH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  FH_HIP(ctx, hipMemcpy(kv_cache(ctx, layer, which) + (uint64_t)page * elements, data, elements * 2,
                        hipMemcpyHostToDevice));
  return FH_OK;
}

// Attention blocks of a prefill chunk: runs of rows of one sequence at
// consecutive positions whose page lists extend one another (so the block's
// last row's table serves every row of it), at most attention_block_rows()
// rows each, stored as first row | rows << 16. Longest first: a block reads
// the pages up to its last row's position, and workgroups are dispatched in
// block order, so the short ones fill the tail.
uint32_t prefill_blocks(const fh_ctx* ctx, const fh_row* rows, uint32_t nrows, uint32_t* blocks) {
  const uint32_t bq = fh::attention_block_rows(ctx->md.query_heads, ctx->md.kv_heads);
  uint32_t nblocks = 0;
  for (uint32_t i = 0; i < nrows;) {
    uint32_t j = i + 1;
    while (j < nrows && j - i < bq && rows[j].sequence == rows[i].sequence &&
           rows[j].position == rows[j - 1].position + 1 && rows[j].page_count >= rows[j - 1].page_count &&
           std::memcmp(rows[j].pages, rows[j - 1].pages, (size_t)rows[j - 1].page_count * 4) == 0)
      ++j;
    blocks[nblocks++] = i | ((j - i) << 16);  // i < 16384, j - i <= 64
    i = j;
  }
  std::stable_sort(blocks, blocks + nblocks, [&](uint32_t a, uint32_t b) {
    return rows[(a & 0xffffu) + (a >> 16) - 1].position > rows[(b & 0xffffu) + (b >> 16) - 1].position;
  });
  return nblocks;
}

// Whether no block reads a slot that another block writes: the pages holding
// a block's positions are listed, up to its last position, by no other
// block's last row (the table that block's attention reads). Then each block
// can append its own rows' K/V inside its attention workgroups.
bool prefill_blocks_private(const fh_row* rows, const uint32_t* blocks, uint32_t nblocks) {
  std::unordered_map<uint32_t, uint32_t> writer;  // physical page -> writing block
  for (uint32_t b = 0; b < nblocks; ++b) {
    const uint32_t i = blocks[b] & 0xffffu, n = blocks[b] >> 16;
    const fh_row& last = rows[i + n - 1];
    for (uint32_t pi = rows[i].position / 16; pi <= last.position / 16; ++pi) {
      const auto ins = writer.emplace(last.pages[pi], b);
      if (!ins.second && ins.first->second != b) return false;
    }
  }
  for (uint32_t b = 0; b < nblocks; ++b) {
    const uint32_t i = blocks[b] & 0xffffu, n = blocks[b] >> 16;
    const fh_row& last = rows[i + n - 1];
    for (uint32_t pi = 0; pi <= last.position / 16; ++pi) {
      const auto it = writer.find(last.pages[pi]);
      if (it != writer.end() && it->second != b) return false;
    }
  }
  return true;
}

// Enqueues (or, dry, only counts) the launches of a prefill chunk of R rows
// with nout output rows, whose metadata (tokens, positions, output rows,
// nblocks attention blocks, page tables) is already in pre.d_meta.
hipError_t enqueue_prefill(fh_ctx* ctx, uint32_t R, uint32_t nout, uint32_t nblocks, bool blocks_private,
                           uint64_t* launches, bool dry = false) {
  const fh_model_desc& md = ctx->md;
  const fh_ctx_options& op = ctx->opt;
  auto& p = ctx->pre;
  const uint32_t P = op.prefill_rows, stride = op.page_table_stride;
  const uint32_t H = md.hidden, QH = md.query_heads, KVH = md.kv_heads, Q = QH * 128, I = md.intermediate,
                 V = md.vocabulary, C = op.context_tokens, pages = op.physical_pages;
  hipStream_t s = ctx->stream;
  const uint32_t* d_tok = p.d_meta;
  const uint32_t* d_pos = p.d_meta + P;
  const uint32_t* d_out = p.d_meta + 2 * P;
  const uint32_t* d_blocks = p.d_meta + 2 * P + kMaxPrefillOutputs;
  const uint32_t* d_tab = p.d_meta + 3 * P + kMaxPrefillOutputs;
  Enq q{ctx, dry};
  if (!dry) (void)hipGetLastError();
  uint32_t* err = ctx->err;
  uint64_t n = 0;
  auto L = [&](uint32_t cls, auto&& f) {
    q.run(cls, f);
    ++n;
  };
  // The fused QKV epilogue needs the 256 x 256-block projection kernel.
  const bool fused_qkv = R > 256 && ctx->nqkv % 256 == 0 && fh::act_mtiles(R) % 16 == 0;
  // Chunks of up to kPanelRows rows (a speculative verify) write split-K
  // partials for QKV, O and down: the QK-norm, the post-attention norm and
  // the next layer's input norm (after the last layer the final norm, whose
  // output is unused here) fold them, as in a decode step. Larger chunks
  // keep the residual in the projection epilogues.
  const bool split_k = R <= fh::kPanelRows;
  const uint32_t sq = R <= kMaxRows ? ctx->s_qkv : p.s_qkv, so = R <= kMaxRows ? ctx->s_o : p.s_o,
                 sd = R <= kMaxRows ? ctx->s_down : p.s_down;
  // Split-K chunks whose blocks write no slot another block reads run the
  // QK-norm, RoPE and KV append inside the attention workgroups (one launch
  // fewer per layer).
  const bool qkn_blocks = split_k && !fused_qkv && blocks_private &&
                          fh::attention_blocks_qkn_supported(QH, KVH, sq);
  L(FH_KC_EMBEDDING, [&] { return fh::launch_clear_word(err, s); });
  L(FH_KC_EMBEDDING, [&] { return fh::launch_embedding(d_tok, ctx->embed, p.hidden, R, H, V, err, s); });
  for (uint32_t l = 0; l < md.layers; ++l) {
    const LayerWeights& W = ctx->layers[l];
    uint16_t* kc = kv_cache(ctx, l, 0);
    uint16_t* vc = kv_cache(ctx, l, 1);
    if (!split_k || l == 0)
      L(FH_KC_RMSNORM, [&] {
        return fh::launch_residual_rmsnorm(p.hidden, nullptr, 0, W.in_norm, p.xn, 1, R, H, md.rms_epsilon, err, s);
      });
    if (fused_qkv) {
      // QK-norm, RoPE and the KV append run in the projection's epilogue.
      const fh::QkvRopeArgs qa{W.q_norm, W.k_norm, ctx->cos_t, ctx->sin_t, d_pos, d_tab, p.qrot, kc, vc,
                               QH,       KVH,      stride,     pages,      C,     md.rms_epsilon, err};
      L(FH_KC_QKV_GEMM, [&] { return fh::launch_gemm_qkv_rope(p.xn, W.qkv, R, ctx->nqkv, H, qa, s); });
    } else {
      L(FH_KC_QKV_GEMM, [&] {
        return split_k ? fh::launch_gemm(p.xn, W.qkv, R, ctx->nqkv, H, FH_EPI_PARTIAL, sq, nullptr, p.part,
                                         ctx->nqkv, err, s)
                       : fh::launch_gemm_large(p.xn, W.qkv, R, ctx->nqkv, H, FH_EPI_BF16, nullptr, p.qkv,
                                               ctx->nqkv, err, s);
      });
      if (!qkn_blocks)
        L(FH_KC_QKNORM_ROPE_KV, [&] {
          return fh::launch_qknorm_rope_kv(split_k ? nullptr : p.qkv, split_k ? p.part : nullptr, split_k ? sq : 0,
                                           W.q_norm, W.k_norm, ctx->cos_t, ctx->sin_t, d_pos, d_tab, p.qrot, kc, vc,
                                           R, QH, KVH, stride, pages, C, md.rms_epsilon, err, s);
        });
    }
    const fh::AttnQkn qa{p.part, sq, fh::partial_slab_rows(R), W.q_norm, W.k_norm, ctx->cos_t, ctx->sin_t,
                         kc,     vc, md.rms_epsilon};
    L(FH_KC_ATTENTION, [&] {
      return fh::launch_attention_blocks(p.qrot, kc, vc, d_pos, d_tab, d_blocks, nblocks, p.attn, 1, R, QH, KVH,
                                         stride, pages, C, err, s, qkn_blocks ? &qa : nullptr);
    });
    if (split_k) {
      L(FH_KC_O_GEMM, [&] {
        return fh::launch_gemm(p.attn, W.o, R, H, Q, FH_EPI_PARTIAL, so, nullptr, p.part, H, err, s);
      });
      L(FH_KC_RMSNORM, [&] {
        return fh::launch_residual_rmsnorm(p.hidden, p.part, so, W.post_norm, p.xn, 1, R, H, md.rms_epsilon, err,
                                           s);
      });
    } else {
      L(FH_KC_O_GEMM, [&] {
        return fh::launch_gemm_large(p.attn, W.o, R, H, Q, FH_EPI_RESIDUAL, p.hidden, p.hidden, H, err, s);
      });
      L(FH_KC_RMSNORM, [&] {
        return fh::launch_residual_rmsnorm(p.hidden, nullptr, 0, W.post_norm, p.xn, 1, R, H, md.rms_epsilon, err,
                                           s);
      });
    }
    L(FH_KC_GATE_UP_GEMM, [&] {
      return fh::launch_gemm_large(p.xn, W.gu, R, 2 * I, H, FH_EPI_SWIGLU, nullptr, p.act, I, err, s);
    });
    if (split_k) {
      const uint16_t* next_norm = l + 1 < md.layers ? ctx->layers[l + 1].in_norm : ctx->final_norm;
      L(FH_KC_DOWN_GEMM, [&] {
        return fh::launch_gemm(p.act, W.down, R, H, I, FH_EPI_PARTIAL, sd, nullptr, p.part, H, err, s);
      });
      L(FH_KC_RMSNORM, [&] {
        return fh::launch_residual_rmsnorm(p.hidden, p.part, sd, next_norm, p.xn, 1, R, H, md.rms_epsilon, err, s);
      });
    } else {
      L(FH_KC_DOWN_GEMM, [&] {
        return fh::launch_gemm_large(p.act, W.down, R, H, I, FH_EPI_RESIDUAL, p.hidden, p.hidden, H, err, s);
      });
    }
    if (ctx->capture)
      L(FH_KC_RMSNORM, [&] {
        return fh::launch_copy_u16(p.hidden, ctx->capture + (uint64_t)l * ctx->capture_rows * H, (uint64_t)R * H, s);
      });
  }
  if (nout) {
    L(FH_KC_RMSNORM, [&] { return fh::launch_gather_rows(p.hidden, d_out, p.out_hidden, nout, H, s); });
    L(FH_KC_RMSNORM, [&] {
      return fh::launch_residual_rmsnorm(p.out_hidden, nullptr, 0, ctx->final_norm, p.out_xn, 1, nout, H,
                                         md.rms_epsilon, err, s);
    });
    L(FH_KC_HEAD_GEMM, [&] {
      return nout <= kMaxRows
                 ? fh::launch_gemm(p.out_xn, ctx->head, nout, V, H, FH_EPI_F32, 1, nullptr, p.logits, V, err, s)
                 : fh::launch_gemm_large(p.out_xn, ctx->head, nout, V, H, FH_EPI_F32, nullptr, p.logits, V, err, s);
    });
    L(FH_KC_ARGMAX, [&] { return fh::launch_argmax(p.logits, nout, V, p.argmax_scratch, p.choices, err, s); });
    ++n;  // argmax is two launches
  }
  *launches = n;
  if (!dry && q.first_error != hipSuccess)
    ctx->launch_detail = std::string(" (kernel class ") + std::to_string(q.first_error_class) + ", launch " +
                         std::to_string(q.first_error_launch) + ")";
  return dry ? hipSuccess : q.first_error;
}

// A prefill chunk (row_capacity < nrows <= prefill_rows), launched eagerly:
// the decode path's op order (batched.rs:1746-2454). Up to 256 rows (a
// speculative verify) the projections are the panel GEMM with split-K
// partials folded by the norms, as in a decode step; beyond that the
// compute-bound 256 x 256-block kernel with the residual (and, for QKV, the
// QK-norm, RoPE and KV append) in its epilogues. Attention runs over blocks
// of consecutive rows of one sequence (each K/V page read once per block),
// and the final norm + FP32 head + argmax over the requested output rows
// only.
fh_status run_prefill(fh_ctx* ctx, uint64_t batch_id, const fh_row* rows, uint32_t nrows,
                      const uint32_t* output_rows, uint32_t nout, uint32_t* choices_out) {
  const fh_model_desc& md = ctx->md;
  const fh_ctx_options& op = ctx->opt;
  auto& p = ctx->pre;
  const uint32_t P = op.prefill_rows, stride = op.page_table_stride;
  const uint32_t QH = md.query_heads, KVH = md.kv_heads, V = md.vocabulary;
  uint32_t* tok = p.h_meta;
  uint32_t* pos = p.h_meta + P;
  uint32_t* outs = p.h_meta + 2 * P;
  uint32_t* blocks = p.h_meta + 2 * P + kMaxPrefillOutputs;
  uint32_t* tab = p.h_meta + 3 * P + kMaxPrefillOutputs;
  for (uint32_t i = 0; i < nrows; ++i) {
    tok[i] = rows[i].token;
    pos[i] = rows[i].position;
    uint32_t* t = tab + (uint64_t)i * stride;
    std::memcpy(t, rows[i].pages, rows[i].page_count * 4);
    std::fill(t + rows[i].page_count, t + stride, 0xffffffffu);
  }
  for (uint32_t i = 0; i < nout; ++i) outs[i] = output_rows[i];
  const uint32_t nblocks = prefill_blocks(ctx, rows, nrows, blocks);
  const bool priv = nrows <= fh::kPanelRows && prefill_blocks_private(rows, blocks, nblocks);
  auto poison = [&](fh_status s2, const std::string& msg) {
    ctx->poisoned = true;
    return fail(ctx, s2, msg);
  };
  hipStream_t s = ctx->stream;
  uint32_t* err = ctx->err;
  const uint64_t meta_bytes = (3ull * P + kMaxPrefillOutputs + (uint64_t)nrows * stride) * 4;
  hipError_t e = hipMemcpyAsync(p.d_meta, p.h_meta, meta_bytes, hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return poison(FH_ERR_DEVICE, std::string("metadata upload: ") + hipGetErrorString(e));
  hipEventRecord(ctx->ev_begin, s);
  if (ctx->profiling) ctx->prof_launches.clear();
  uint64_t n = 0;
  e = enqueue_prefill(ctx, nrows, nout, nblocks, priv, &n);
  if (e != hipSuccess) return poison(FH_ERR_DEVICE, std::string("launch: ") + hipGetErrorString(e) + ctx->launch_detail);
  hipEventRecord(ctx->ev_end, s);
  if (nout) e = hipMemcpyAsync(p.h_out, p.choices, nout * 4, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipMemcpyAsync(p.h_out + kMaxPrefillOutputs, err, 4, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return poison(FH_ERR_DEVICE, std::string("step: ") + hipGetErrorString(e));
  hipEventElapsedTime(&ctx->last_ms, ctx->ev_begin, ctx->ev_end);
  if (ctx->profiling) collect_profile(ctx);
  ctx->last_rows = nout;
  ctx->last_batch_rows = nrows;
  ctx->last_logits = p.logits;
  ctx->last_was_prefill = true;
  const uint32_t errw = p.h_out[kMaxPrefillOutputs];
  if (errw != 0) return poison(FH_ERR_NONFINITE, "device rejected the step:" + error_bits(errw));
  for (uint32_t i = 0; i < nout; ++i) {
    const uint32_t c = p.h_out[i];
    if (c >= V) return poison(FH_ERR_NONFINITE, "batched GPU choice outside vocabulary");
    choices_out[i] = c;
  }
  ctx->last_batch = batch_id;
  ctx->dispatches += n;
  return FH_OK;
}

// Polls the per-row words the step's last launch sets once its choices are
// stored (coherent pinned memory), so the calling thread is running when the
// step ends instead of being woken from a blocking wait: measured on MI355X,
// waking from hipStreamSynchronize added 50-180 us to a 3.3 ms step. The
// thread spins for at most kChoicesSpinMs; the stream synchronize that
// follows then waits, and reports errors, as before.
constexpr int kChoicesSpinMs = 100;

void await_choices(const uint32_t* done, uint32_t rows) {
  const auto t0 = std::chrono::steady_clock::now();
  for (uint32_t i = 0; i < rows; ++i)
    while (__atomic_load_n(done + i, __ATOMIC_ACQUIRE) == 0u) {
      if (std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(kChoicesSpinMs)) return;
      __builtin_ia32_pause();
    }
}

fh_status fh_execute_batch(fh_ctx* ctx, uint64_t batch_id, const fh_row* rows, uint32_t nrows,
                           const uint32_t* output_rows, uint32_t nout, uint32_t* choices_out) {
  if (!ctx) return FH_ERR_INVALID_ARGUMENT;
  if (nout && (!output_rows || !choices_out)) return fail(ctx, FH_ERR_INVALID_ARGUMENT, "null output buffers");
  fh_status st = validate_batch(ctx, batch_id, rows, nrows, output_rows, nout);
  if (st != FH_OK) return st;
  if (nrows > ctx->opt.row_capacity) return run_prefill(ctx, batch_id, rows, nrows, output_rows, nout, choices_out);

  const uint32_t cap = ctx->opt.row_capacity, stride = ctx->opt.page_table_stride;
  uint32_t* tok = ctx->h_meta;
  uint32_t* pos = ctx->h_meta + cap;
  uint32_t* tab = ctx->h_meta + 2 * cap;
  for (uint32_t i = 0; i < nrows; ++i) {
    tok[i] = rows[i].token;
    pos[i] = rows[i].position;
    uint32_t* t = tab + (uint64_t)i * stride;
    std::memcpy(t, rows[i].pages, rows[i].page_count * 4);
    std::fill(t + rows[i].page_count, t + stride, 0xffffffffu);
  }
  auto poison = [&](fh_status s2, const std::string& msg) {
    ctx->poisoned = true;
    return fail(ctx, s2, msg);
  };
  hipStream_t s = ctx->stream;
  hipError_t e = hipSuccess;
  uint32_t* done = ctx->h_out + cap + 1;
  for (uint32_t i = 0; i < nrows; ++i) __atomic_store_n(done + i, 0u, __ATOMIC_RELAXED);
  hipEventRecord(ctx->ev_begin, s);
  uint64_t launches = 0;
  if (ctx->profiling) ctx->prof_launches.clear();
  if (ctx->opt.use_graphs && !ctx->profiling) {
    // One graph per row count and per form of the attention stage.
    const uint32_t key = nrows | (step_runs_qkn(ctx, nrows) ? 1u << 16 : 0u);
    auto it = ctx->graphs.find(key);
    if (it == ctx->graphs.end()) {
      hipGraph_t g = nullptr;
      hipGraphExec_t ge = nullptr;
      e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
      if (e == hipSuccess) {
        hipError_t le = enqueue_step(ctx, nrows, &launches);
        e = hipStreamEndCapture(s, &g);
        if (e == hipSuccess && le != hipSuccess) e = le;
      }
      if (e == hipSuccess) e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
      if (e != hipSuccess) {
        if (g) hipGraphDestroy(g);
        return poison(FH_ERR_DEVICE, std::string("graph capture: ") + hipGetErrorString(e));
      }
      ctx->graph_defs.push_back(g);
      it = ctx->graphs.emplace(key, fh_ctx::StepGraph{ge, launches}).first;
    }
    launches = it->second.launches;  // a replay issues what its capture recorded
    e = hipGraphLaunch(it->second.exec, s);
  } else {
    e = enqueue_step(ctx, nrows, &launches);
  }
  if (e != hipSuccess) return poison(FH_ERR_DEVICE, std::string("launch: ") + hipGetErrorString(e) + ctx->launch_detail);
  hipEventRecord(ctx->ev_end, s);
  // The step's first launch read h_meta and its last one wrote h_out.
  await_choices(done, nrows);
  e = hipStreamSynchronize(s);
  if (e != hipSuccess) return poison(FH_ERR_DEVICE, std::string("step: ") + hipGetErrorString(e));
  hipEventElapsedTime(&ctx->last_ms, ctx->ev_begin, ctx->ev_end);
  if (ctx->profiling) collect_profile(ctx);
  ctx->last_rows = nrows;
  ctx->last_batch_rows = nrows;
  ctx->last_qkn = step_runs_qkn(ctx, nrows);
  ctx->last_logits = ctx->logits;
  ctx->last_was_prefill = false;
  const uint32_t errw = ctx->h_out[cap];
  if (errw != 0) return poison(FH_ERR_NONFINITE, "device rejected the step:" + error_bits(errw));
  for (uint32_t i = 0; i < nout; ++i) {
    const uint32_t c = ctx->h_out[output_rows[i]];
    if (c >= ctx->md.vocabulary) return poison(FH_ERR_NONFINITE, "batched GPU choice outside vocabulary");
    choices_out[i] = c;
  }
  ctx->last_batch = batch_id;
  ctx->dispatches += launches;
  return FH_OK;
}

fh_status fh_read_logits(fh_ctx* ctx, float* out, uint64_t elements) {
  if (!ctx || !out || elements > (uint64_t)ctx->last_rows * ctx->md.vocabulary)
    return fail(ctx, FH_ERR_INVALID_ARGUMENT, "bad logits request");
  FH_HIP(ctx, hipMemcpy(out, ctx->last_logits, elements * 4, hipMemcpyDeviceToHost));
  return FH_OK;
}

fh_status fh_read_hidden(fh_ctx* ctx, uint32_t layer, uint16_t* out, uint64_t elements) {
  if (!ctx || !out || !ctx->capture || layer >= ctx->md.layers ||
      elements > (uint64_t)ctx->last_batch_rows * ctx->md.hidden)
    return fail(ctx, FH_ERR_INVALID_ARGUMENT, "bad hidden-state request (capture_hidden off?)");
  FH_HIP(ctx, hipMemcpy(out, ctx->capture + (uint64_t)layer * ctx->capture_rows * ctx->md.hidden, elements * 2,
                        hipMemcpyDeviceToHost));
  return FH_OK;
}

fh_status fh_expected_dispatch_count(fh_ctx* ctx, uint64_t batch_id, const fh_row* rows, uint32_t nrows,
                                     const uint32_t* output_rows, uint32_t nout, uint64_t* count) {
  if (!ctx || !count) return FH_ERR_INVALID_ARGUMENT;
  if (nout && !output_rows) return fail(ctx, FH_ERR_INVALID_ARGUMENT, "null output rows");
  // The batch is checked as fh_execute_batch checks it (which also decides
  // whether its rows' written slots are private, one input of the policy),
  // then the step's own enqueue code runs without launching anything.
  fh_status st = validate_batch(ctx, batch_id, rows, nrows, output_rows, nout);
  if (st != FH_OK) return st;
  uint64_t n = 0;
  if (nrows > ctx->opt.row_capacity) {
    std::vector<uint32_t> blocks(nrows);
    const uint32_t nblocks = prefill_blocks(ctx, rows, nrows, blocks.data());
    const bool priv = nrows <= fh::kPanelRows && prefill_blocks_private(rows, blocks.data(), nblocks);
    enqueue_prefill(ctx, nrows, nout, nblocks, priv, &n, true);
  }
  else
    enqueue_step(ctx, nrows, &n, true);
  *count = n;
  return FH_OK;
}

uint32_t fh_row_capacity(const fh_ctx* ctx) { return ctx ? ctx->opt.row_capacity : 0; }
uint64_t fh_dispatch_count(const fh_ctx* ctx) { return ctx ? ctx->dispatches : 0; }
float fh_last_step_ms(const fh_ctx* ctx) { return ctx ? ctx->last_ms : 0.f; }

fh_status fh_set_profiling(fh_ctx* ctx, uint32_t enabled) {
  if (!ctx) return FH_ERR_INVALID_ARGUMENT;
  ctx->profiling = enabled != 0;
  if (ctx->profiling && ctx->prof_events.empty()) {
    const uint64_t need = 2 * (12 + 12ull * ctx->md.layers);
    for (uint64_t i = 0; i < need; ++i) {
      hipEvent_t ev;
      FH_HIP(ctx, hipEventCreate(&ev));
      ctx->prof_events.push_back(ev);
    }
  }
  return FH_OK;
}

fh_status fh_time_attention(fh_ctx* ctx, uint32_t reps, float* avg_ms) {
  if (!ctx || !avg_ms || reps == 0 || reps > 1000) return FH_ERR_INVALID_ARGUMENT;
  if (ctx->poisoned) return fail(ctx, FH_ERR_POISONED, "runtime poisoned by an earlier failure");
  if (ctx->last_was_prefill || ctx->last_rows == 0) return fail(ctx, FH_ERR_STATE, "no decode batch to time");
  const fh_model_desc& md = ctx->md;
  const fh_ctx_options& op = ctx->opt;
  const uint32_t R = ctx->last_rows, cap = op.row_capacity, l = md.layers - 1;
  const uint32_t* d_pos = ctx->d_meta + cap;
  const uint32_t* d_tab = ctx->d_meta + 2 * cap;
  hipStream_t s = ctx->stream;
  auto launch = [&] {
    const uint32_t split = fh::attn_split_pages(R, md.query_heads, op.context_tokens);
    const bool fuse = fh::attn_fuse_merge(R, md.kv_heads, op.context_tokens, split);
    // The attention kernel class of the step: the partition launch (with the
    // merge when the step fuses it; the merge launch is a class of its own).
    // A step that ran the QK-norm/KV append inside attention is timed in
    // that form (it rewrites the same new slots with the same values).
    const fh::AttnQkn qa = step_qkn_args(ctx, l);
    return fh::launch_attention_partial(ctx->qrot, kv_cache(ctx, l, 0), kv_cache(ctx, l, 1), d_pos, d_tab,
                                        ctx->attn_part, ctx->attn, 1, 0, R, R, md.query_heads, md.kv_heads,
                                        op.page_table_stride, op.physical_pages, op.context_tokens, split,
                                        fuse ? ctx->attn_count : nullptr, ctx->err, s, ctx->last_qkn ? &qa : nullptr);
  };
  hipEvent_t a = nullptr, b = nullptr;
  (void)hipGetLastError();
  hipError_t e = hipEventCreate(&a);
  if (e == hipSuccess) e = hipEventCreate(&b);
  if (e == hipSuccess) e = launch();  // warm: same inputs, so the same outputs as the step wrote
  if (e == hipSuccess) e = hipEventRecord(a, s);
  for (uint32_t i = 0; i < reps && e == hipSuccess; ++i) e = launch();
  if (e == hipSuccess) e = hipEventRecord(b, s);
  if (e == hipSuccess) e = hipEventSynchronize(b);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
  if (a) hipEventDestroy(a);
  if (b) hipEventDestroy(b);
  if (e != hipSuccess) {
    ctx->poisoned = true;
    return fail(ctx, FH_ERR_DEVICE, std::string("attention timing: ") + hipGetErrorString(e));
  }
  *avg_ms = ms / (float)reps;
  return FH_OK;
}

fh_status fh_kernel_class_ms(const fh_ctx* ctx, uint32_t cls, float* ms, uint32_t* launches) {
  if (!ctx || cls >= FH_KC_COUNT || !ms || !launches) return FH_ERR_INVALID_ARGUMENT;
  *ms = ctx->class_ms[cls];
  *launches = ctx->class_launches[cls];
  return FH_OK;
}

}  // extern "C"
