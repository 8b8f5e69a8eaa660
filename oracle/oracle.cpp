// Test infrastructure only: the CPU oracle for the Qwen3 forward-pass hot path.
//
// A plain C++ restatement of the reference's *serial* scalar semantics — the
// v1 kernel roots of device/qwen3-all-kernels-v1 and the host arithmetic of
// adapters/m1-engineering-execution-v1 — used by tests/, the smoke check and
// bench.py's CPU baseline to check the HIP library. Nothing in the product
// path links or calls this file.
//
// Every reduction runs in the reference's order (ascending index, one
// rounding per product and per sum; build with -ffp-contract=off), so the
// result does not depend on the OpenMP thread count. exp/sqrt are the host
// libm's: the reference's device exp (OCML) and the host libm can differ in
// the last ulp, which the tests treat as tolerance, not parity.
//
// Pinning: every function below is checked in tests/test_oracle.py against
// the reference's known-answer vectors or a closed form; see the list in the
// header comment of that file.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include <omp.h>

#include "../include/ferric_synth.h"

namespace {

inline float widen(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

inline uint32_t bits_of(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}

// device/qwen3-gemm-v1/tests/reference.rs:3-11 (RNE, NaN quieted with |0x40).
inline uint16_t narrow(float v) {
  uint32_t b = bits_of(v);
  if ((b & 0x7f800000u) == 0x7f800000u && (b & 0x007fffffu) != 0u) return (uint16_t)((b >> 16) | 0x0040u);
  return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

inline bool finite(float v) { return std::isfinite(v); }
inline bool finite_bf16(uint16_t b) { return (b & 0x7f80u) != 0x7f80u; }

constexpr uint32_t kScaleBits = 0x3db504f3u;  // paged_decode.rs:31-35

}  // namespace

extern "C" {

uint16_t orc_bf16_from_f32(float v) { return narrow(v); }
float orc_f32_from_bf16(uint16_t b) { return widen(b); }

// Serial FP32 sum of squares in ascending order (rmsnorm.rs:421-438;
// device/qwen3-rmsnorm-v1/tests/reference.rs:33-38).
float orc_square_sum(const uint16_t* x, uint32_t n) {
  float sum = 0.0f;
  for (uint32_t i = 0; i < n; ++i) {
    float v = widen(x[i]);
    float sq = v * v;
    sum = sum + sq;
  }
  return sum;
}

// Normalize-then-round, weight, round again (rmsnorm.rs:486-503;
// device/qwen3-rmsnorm-v1/tests/reference.rs:19-31). Returns 0x7fff... on
// the reference's rejection (nonfinite intermediate): 0xffffffff.
uint32_t orc_norm_weight(float normalized, uint16_t weight) {
  float narrowed = widen(narrow(normalized));
  if (!finite(normalized) || !finite(narrowed)) return 0xffffffffu;
  float w = widen(weight);
  float weighted = narrowed * w;
  uint16_t out = narrow(weighted);
  if (!finite(w) || !finite(weighted) || !finite_bf16(out)) return 0xffffffffu;
  return out;
}

// qwen3_rmsnorm_v1 (device/qwen3-all-kernels-v1/src/rmsnorm.rs:380-526), as
// restated by device/qwen3-rmsnorm-v1/tests/reference.rs:94-180.
// behavior 0: pure; behavior 1: residual-fused (fused_out = bf16(x + r), the
// norm uses the unrounded f32 sum). Returns 0, or 1 where the reference traps.
int orc_rmsnorm(const uint16_t* input, const uint16_t* residual, const uint16_t* weight, uint32_t rows,
                uint32_t width, float eps, uint32_t behavior, uint16_t* fused_out, uint16_t* norm_out) {
  const bool fused = behavior == 1;
  for (uint32_t r = 0; r < rows; ++r) {
    const uint64_t base = (uint64_t)r * width;
    float sum = 0.0f;
    for (uint32_t c = 0; c < width; ++c) {
      float x = widen(input[base + c]);
      if (!finite(x)) return 1;
      if (fused) {
        float rv = widen(residual[base + c]);
        x = x + rv;
        if (!finite(rv) || !finite(x)) return 1;
      }
      float sq = x * x;
      float next = sum + sq;
      if (!finite(sq) || !finite(next)) return 1;
      sum = next;
    }
    // (pure mode: this loop is orc_square_sum plus the reference's per-step
    // finiteness checks)
    float mean_square = sum / (float)width;
    float stabilized = mean_square + eps;
    float denominator = std::sqrt(stabilized);
    float inverse = 1.0f / denominator;
    if (!finite(mean_square) || !finite(stabilized) || stabilized <= 0.f || !finite(denominator) ||
        denominator <= 0.f || !finite(inverse))
      return 1;
    for (uint32_t c = 0; c < width; ++c) {
      float x = widen(input[base + c]);
      if (fused) {
        float f = x + widen(residual[base + c]);
        uint16_t nf = narrow(f);
        if (!finite_bf16(nf)) return 1;
        fused_out[base + c] = nf;
        x = f;
      }
      float normalized = x * inverse;
      uint32_t out = orc_norm_weight(normalized, weight[c]);
      if (out == 0xffffffffu) return 1;
      norm_out[base + c] = (uint16_t)out;
    }
  }
  return 0;
}

// ferric_qwen3_gemm_reference_bf16_f32_bf16_v1 (gemm.rs:161-337;
// device/qwen3-gemm-v1/tests/reference.rs:17-46): C[m][n] = bf16(sum_k
// a[m][k] * b[n][k] (+ C_old if beta_one)), FP32 ascending-k accumulation.
// out_f32 != NULL selects the FP32-output LM head (no narrowing;
// device/qwen3-tp-fp32-head32-kernels-v8/src/projection.rs:66).
void orc_gemm(const uint16_t* a, const uint16_t* b, const uint16_t* prior_c, uint32_t m, uint32_t n, uint32_t k,
              uint32_t beta_one, uint16_t* out, float* out_f32) {
  // Activations transposed to [k][m] floats so each output row's serial
  // chain is one SIMD lane: lane j computes acc_j = acc_j + a[j][k] * w[k].
  const uint32_t mp = (m + 7) & ~7u;
  std::vector<float> at((uint64_t)k * mp, 0.f);
  for (uint32_t r = 0; r < m; ++r)
    for (uint32_t c = 0; c < k; ++c) at[(uint64_t)c * mp + r] = widen(a[(uint64_t)r * k + c]);
#pragma omp parallel
  {
    std::vector<float> acc(mp);
    std::vector<float> w(k);
#pragma omp for schedule(static)
    for (int64_t col = 0; col < (int64_t)n; ++col) {
      const uint16_t* brow = b + (uint64_t)col * k;
      for (uint32_t c = 0; c < k; ++c) w[c] = widen(brow[c]);
      std::fill(acc.begin(), acc.end(), 0.f);
      float* accp = acc.data();
      for (uint32_t c = 0; c < k; ++c) {
        const float wc = w[c];
        const float* ar = at.data() + (uint64_t)c * mp;
        for (uint32_t j = 0; j < mp; ++j) {
          float product = ar[j] * wc;
          accp[j] = accp[j] + product;
        }
      }
      for (uint32_t r = 0; r < m; ++r) {
        const uint64_t o = (uint64_t)r * n + col;
        if (out_f32) {
          out_f32[o] = acc[r];
        } else {
          float v = acc[r];
          if (beta_one) v = v + widen(prior_c[o]);
          out[o] = narrow(v);
        }
      }
    }
  }
}

// Serial-in-groups-of-4 variant (gemm.rs:355 `a4`), equal to orc_gemm for
// every input because the order of additions is unchanged.
void orc_gemm_a4(const uint16_t* a, const uint16_t* b, const uint16_t* prior_c, uint32_t m, uint32_t n, uint32_t k,
                 uint32_t beta_one, uint16_t* out) {
  for (uint32_t r = 0; r < m; ++r)
    for (uint32_t col = 0; col < n; ++col) {
      float acc = 0.f;
      for (uint32_t c = 0; c < k; c += 4)
        for (uint32_t o = 0; o < 4; ++o) {
          float product = widen(a[(uint64_t)r * k + c + o]) * widen(b[(uint64_t)col * k + c + o]);
          acc = acc + product;
        }
      if (beta_one) acc = acc + widen(prior_c[(uint64_t)r * n + col]);
      out[(uint64_t)r * n + col] = narrow(acc);
    }
}

// ---- the reference's wave-order profiles (a second legal reduction order) ----
// The serial functions above are the v1 semantics. The reference's resident
// decode path reassociates the same sums across a 64-lane wave:
//   * wave GEMV (device/qwen3-tp-batch32-kernels-v5/src/projection.rs:15-137,
//     partial form :142): lane l accumulates the products k = 64 s + l for
//     s = 0, 1, ... in order, then reduce_sum_f32::<64> combines the lanes;
//   * wave RMSNorm (device/qwen3-tp-wave-rmsnorm-kernels-v15/src/rmsnorm.rs:
//     60-75): lane l accumulates x[l + 64 c]^2 for c = 0, 1, ..., then the
//     same reduction;
//   * wave attention (device/qwen3-tp-wave-query-hoist-kernels-v14/src/
//     attention.rs:174-217): lane l forms q[l] k[l] + q[l+64] k[l+64], then
//     the reduction gives the score; the online softmax is the serial one.
// reduce_sum_f32::<64> is fe2o3's (not in the reference tree); it is taken
// here as the xor butterfly v += lane(v ^ off) for off = 32, 16, ..., 1,
// which leaves every lane with the same value because each addition is
// commutative. These give the spread two legal orders of the reference's own
// arithmetic produce end to end, the yardstick for a third order's (the
// GPU's) drift.
static float wave_reduce64(float* v) {
  float t[64];
  for (int off = 32; off > 0; off >>= 1) {
    for (int l = 0; l < 64; ++l) t[l] = v[l] + v[l ^ off];
    std::memcpy(v, t, sizeof(t));
  }
  return v[0];
}

// C = A W^T in wave-GEMV order (k % 64 == 0). out (bf16, one RNE) or out_f32.
void orc_gemm_wave(const uint16_t* a, const uint16_t* b, uint32_t m, uint32_t n, uint32_t k, uint16_t* out,
                   float* out_f32) {
  std::vector<float> af((uint64_t)m * k);
  for (uint64_t i = 0; i < (uint64_t)m * k; ++i) af[i] = widen(a[i]);
  const uint32_t steps = k / 64;
#pragma omp parallel
  {
    std::vector<float> w(k);
    float lanes[64];
#pragma omp for schedule(static)
    for (int64_t col = 0; col < (int64_t)n; ++col) {
      const uint16_t* brow = b + (uint64_t)col * k;
      for (uint32_t c = 0; c < k; ++c) w[c] = widen(brow[c]);
      for (uint32_t r = 0; r < m; ++r) {
        const float* ar = af.data() + (uint64_t)r * k;
        for (int l = 0; l < 64; ++l) lanes[l] = 0.f;
        for (uint32_t st = 0; st < steps; ++st) {
          const float* as = ar + (uint64_t)st * 64;
          const float* ws = w.data() + (uint64_t)st * 64;
          for (int l = 0; l < 64; ++l) {
            float product = as[l] * ws[l];
            lanes[l] = lanes[l] + product;
          }
        }
        const float sum = wave_reduce64(lanes);
        const uint64_t o = (uint64_t)r * n + col;
        if (out_f32)
          out_f32[o] = sum;
        else
          out[o] = narrow(sum);
      }
    }
  }
}

// Wave-order sum of squares of one row (width % 64 == 0): lane l adds
// x[l + 64 c]^2 in ascending c, then the 64-lane butterfly.
float orc_square_sum_wave(const uint16_t* x, uint32_t width) {
  float lanes[64];
  for (int l = 0; l < 64; ++l) {
    float partial = 0.f;
    for (uint32_t c = (uint32_t)l; c < width; c += 64) {
      const float v = widen(x[c]);
      const float sq = v * v;
      partial = partial + sq;
    }
    lanes[l] = partial;
  }
  return wave_reduce64(lanes);
}

// Pure RMSNorm with the wave-order sum of squares (width % 64 == 0); the
// normalize-and-weight step is the serial one. Returns 1 where the reference traps.
int orc_rmsnorm_wave(const uint16_t* input, const uint16_t* weight, uint32_t rows, uint32_t width, float eps,
                     uint16_t* norm_out) {
  for (uint32_t r = 0; r < rows; ++r) {
    const uint64_t base = (uint64_t)r * width;
    float lanes[64];
    for (int l = 0; l < 64; ++l) {
      float partial = 0.f;
      for (uint32_t c = (uint32_t)l; c < width; c += 64) {
        const float x = widen(input[base + c]);
        const float sq = x * x;
        const float next = partial + sq;
        if (!finite(x) || !finite(sq) || !finite(next)) return 1;
        partial = next;
      }
      lanes[l] = partial;
    }
    const float sum = wave_reduce64(lanes);
    const float mean_square = sum / (float)width;
    const float stabilized = mean_square + eps;
    const float denominator = std::sqrt(stabilized);
    const float inverse = 1.0f / denominator;
    if (!finite(sum) || !finite(mean_square) || !finite(stabilized) || stabilized <= 0.f || !finite(denominator) ||
        denominator <= 0.f || !finite(inverse))
      return 1;
    for (uint32_t c = 0; c < width; ++c) {
      const uint32_t o = orc_norm_weight(widen(input[base + c]) * inverse, weight[c]);
      if (o == 0xffffffffu) return 1;
      norm_out[base + c] = (uint16_t)o;
    }
  }
  return 0;
}

// Pure RMSNorm whose sum of squares is taken exactly: the squares rounded to
// FP32 as the reference forms them (rmsnorm.rs:421-438), summed in double
// (exact to well below an FP32 ulp for rows of up to 8192 squares), rounded
// to FP32 once; the inverse and the normalize-and-weight steps are the serial
// ones. The most accurate reassociation of the reference's sum, so one more
// point of its arithmetic's legal spread. Returns 1 where the reference traps.
int orc_rmsnorm_exact(const uint16_t* input, const uint16_t* weight, uint32_t rows, uint32_t width, float eps,
                      uint16_t* norm_out) {
  for (uint32_t r = 0; r < rows; ++r) {
    const uint64_t base = (uint64_t)r * width;
    double acc = 0.0;
    for (uint32_t c = 0; c < width; ++c) {
      const float x = widen(input[base + c]);
      const float sq = x * x;
      if (!finite(x) || !finite(sq)) return 1;
      acc += (double)sq;
    }
    const float sum = (float)acc;
    const float mean_square = sum / (float)width;
    const float stabilized = mean_square + eps;
    const float denominator = std::sqrt(stabilized);
    const float inverse = 1.0f / denominator;
    if (!finite(sum) || !finite(mean_square) || !finite(stabilized) || stabilized <= 0.f || !finite(denominator) ||
        denominator <= 0.f || !finite(inverse))
      return 1;
    for (uint32_t c = 0; c < width; ++c) {
      const uint32_t o = orc_norm_weight(widen(input[base + c]) * inverse, weight[c]);
      if (o == 0xffffffffu) return 1;
      norm_out[base + c] = (uint16_t)o;
    }
  }
  return 0;
}

// ferric_qwen3_token_embedding_bf16_copy_v1 (gemm.rs:768-853): bit copy;
// returns the first row whose token is out of range + 1, or 0.
uint32_t orc_embedding(const uint32_t* tokens, const uint16_t* weight, uint32_t rows, uint32_t hidden,
                       uint32_t vocab, uint16_t* out) {
  for (uint32_t r = 0; r < rows; ++r) {
    if (tokens[r] >= vocab) return r + 1;
    std::memcpy(out + (uint64_t)r * hidden, weight + (uint64_t)tokens[r] * hidden, (uint64_t)hidden * 2);
  }
  return 0;
}

// rope_bytes (adapters/m1-engineering-execution-v1/src/tp_execution.rs:1440-1450).
void orc_rope_table(uint32_t position, uint32_t theta, float* cos_out, float* sin_out) {
  for (uint32_t pair = 0; pair < 64; ++pair) {
    double inverse_frequency = std::pow((double)theta, -(double)pair / 64.0);
    double angle = (double)position * inverse_frequency;
    cos_out[pair] = (float)std::cos(angle);
    sin_out[pair] = (float)std::sin(angle);
  }
}

// Split-half RoPE pair (rope_kv.rs:168-200; device/qwen3-rope-kv-v1/tests/reference.rs:22-36).
void orc_rope_pair(uint16_t first, uint16_t second, float c, float s, uint16_t* out2) {
  float f = widen(first), g = widen(second);
  float first_cos = f * c;
  float second_sin = g * s;
  float rotated_first = first_cos - second_sin;
  float second_cos = g * c;
  float first_sin = f * s;
  float rotated_second = second_cos + first_sin;
  out2[0] = narrow(rotated_first);
  out2[1] = narrow(rotated_second);
}

// Paged cache element index (rope_kv.rs:340-360; paged_decode.rs:440-470):
// ((physical_page * 16 + token_in_page) * kv_heads + kv_head) * 128 + feature.
uint64_t orc_cache_index(uint32_t physical_page, uint32_t token_in_page, uint32_t kv_heads, uint32_t kv_head,
                         uint32_t feature) {
  return (((uint64_t)physical_page * 16 + token_in_page) * kv_heads + kv_head) * 128 + feature;
}

// qwen3_paged_gqa_decode_bf16_f32_v1 for one query head
// (paged_decode.rs:222-572; device/qwen3-paged-decode-v1/tests/reference.rs:33-121):
// keys 0..=position through `pages`, serial 128-wide dot, score * f32(0x3db504f3),
// online softmax, out = bf16(n / l). Returns 1 where the reference traps.
static int attention_head_ordered(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                  const uint32_t* pages, uint32_t page_count, uint32_t physical_pages,
                                  uint32_t position, uint32_t kv_heads, uint32_t kv_head, uint16_t* out, int order);

int orc_attention_head(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, const uint32_t* pages,
                       uint32_t page_count, uint32_t physical_pages, uint32_t position, uint32_t kv_heads,
                       uint32_t kv_head, uint16_t* out) {
  return attention_head_ordered(q, k_cache, v_cache, pages, page_count, physical_pages, position, kv_heads, kv_head,
                                out, 0);
}

// The same head in the split-context wave-order profile (v21 partitions with
// v14 score dots), below.
int orc_attention_head_wave(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                            const uint32_t* pages, uint32_t page_count, uint32_t physical_pages, uint32_t position,
                            uint32_t kv_heads, uint32_t kv_head, uint16_t* out) {
  return attention_head_ordered(q, k_cache, v_cache, pages, page_count, physical_pages, position, kv_heads, kv_head,
                                out, 1);
}

// Online-softmax state of the keys [begin, end) of one head: t = begin gives
// m = s, l = 1, n = v; later keys m' = max(m, s), l = l e^(m-m') + e^(s-m'),
// n likewise (paged_decode.rs:222-572). order 0: serial 128-wide score dot;
// order 1: the wave-order dot. Returns 1 where the reference traps.
static int attention_span(const float* qf, const uint16_t* k_cache, const uint16_t* v_cache, const uint32_t* pages,
                          uint32_t page_count, uint32_t physical_pages, uint32_t begin, uint32_t end,
                          uint32_t kv_heads, uint32_t kv_head, int order, float* m_out, float* l_out, float* n) {
  float scale;
  std::memcpy(&scale, &kScaleBits, 4);
  float m = 0.f, l = 0.f;
  for (uint32_t t = begin; t < end; ++t) {
    uint32_t lp = t / 16, slot = t % 16;
    if (lp >= page_count) return 1;
    uint32_t phys = pages[lp];
    if (phys >= physical_pages) return 1;
    const uint64_t base = orc_cache_index(phys, slot, kv_heads, kv_head, 0);
    float dot = 0.f;
    if (order == 0) {
      for (int d = 0; d < 128; ++d) {
        float kf = widen(k_cache[base + d]);
        float product = qf[d] * kf;
        float next = dot + product;
        if (!finite(qf[d]) || !finite(kf) || !finite(product) || !finite(next)) return 1;
        dot = next;
      }
    } else {
      float lanes[64];
      for (int ln = 0; ln < 64; ++ln) {
        const float k0 = widen(k_cache[base + ln]), k1 = widen(k_cache[base + ln + 64]);
        const float p0 = qf[ln] * k0, p1 = qf[ln + 64] * k1;
        const float partial = p0 + p1;
        if (!finite(p0) || !finite(p1) || !finite(partial)) return 1;
        lanes[ln] = partial;
      }
      dot = wave_reduce64(lanes);
      if (!finite(dot)) return 1;
    }
    float score = dot * scale;
    if (!finite(score)) return 1;
    if (t == begin) {
      m = score;
      l = 1.f;
      for (int d = 0; d < 128; ++d) {
        n[d] = widen(v_cache[base + d]);
        if (!finite(n[d])) return 1;
      }
    } else {
      float next_max = score > m ? score : m;
      float pw = std::exp(m - next_max);
      float cw = std::exp(score - next_max);
      float next_l = l * pw + cw;
      if (!finite(pw) || !finite(cw) || !finite(next_l) || next_l <= 0.f) return 1;
      for (int d = 0; d < 128; ++d) {
        float v = widen(v_cache[base + d]);
        float nn = n[d] * pw + v * cw;
        if (!finite(v) || !finite(nn)) return 1;
        n[d] = nn;
      }
      m = next_max;
      l = next_l;
    }
  }
  *m_out = m;
  *l_out = l;
  return 0;
}

// order 0: qwen3_paged_gqa_decode_bf16_f32_v1, one serial recurrence over keys
// 0..=position. order 1: the reference's split-context profile
// (device/qwen3-tp-c1-split8-attention-kernels-v21/src/attention.rs:16-213,
// merge :214-308): 8 contiguous partitions of ceil(keys / 8) keys, each its
// own recurrence with wave-order score dots (v14), then the partition states
// merged in ascending order by the same recurrence (a partition's m and l in
// place of a key's score and 1), divided and narrowed once.
static int attention_head_ordered(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                  const uint32_t* pages, uint32_t page_count, uint32_t physical_pages,
                                  uint32_t position, uint32_t kv_heads, uint32_t kv_head, uint16_t* out, int order) {
  float qf[128];
  for (int d = 0; d < 128; ++d) qf[d] = widen(q[d]);
  const uint32_t keys = position + 1;
  float M = 0.f, L = 0.f, N[128];
  if (order == 0) {
    if (attention_span(qf, k_cache, v_cache, pages, page_count, physical_pages, 0, keys, kv_heads, kv_head, 0, &M, &L,
                       N))
      return 1;
  } else {
    const uint32_t span = (keys + 7) / 8;
    for (uint32_t p = 0; p < 8 && p * span < keys; ++p) {
      float m, l, n[128];
      const uint32_t begin = p * span, end = std::min(keys, begin + span);
      if (attention_span(qf, k_cache, v_cache, pages, page_count, physical_pages, begin, end, kv_heads, kv_head, 1,
                         &m, &l, n))
        return 1;
      if (p == 0) {
        M = m;
        L = l;
        std::memcpy(N, n, sizeof(N));
      } else {
        const float next_max = m > M ? m : M;
        const float pw = std::exp(M - next_max);
        const float cw = std::exp(m - next_max);
        L = L * pw + l * cw;
        if (!finite(pw) || !finite(cw) || !finite(L) || L <= 0.f) return 1;
        for (int d = 0; d < 128; ++d) {
          N[d] = N[d] * pw + n[d] * cw;
          if (!finite(N[d])) return 1;
        }
        M = next_max;
      }
    }
  }
  for (int d = 0; d < 128; ++d) {
    float o = N[d] / L;
    uint16_t b = narrow(o);
    if (!finite(o) || !finite_bf16(b)) return 1;
    out[d] = b;
  }
  return 0;
}

// qwen3_swiglu_element_v1 (device/qwen3-all-kernels-v1/src/swiglu.rs:62-101;
// device/qwen3-swiglu-v1/tests/reference.rs:17-40). Returns 1 where the reference traps.
int orc_swiglu(const uint16_t* gate, const uint16_t* up, uint64_t count, uint16_t* out) {
  for (uint64_t i = 0; i < count; ++i) {
    float g = widen(gate[i]), u = widen(up[i]);
    if (!finite(g) || !finite(u)) return 1;
    bool nonneg = g >= 0.0f;
    float e = std::exp(nonneg ? -g : g);
    float denom = 1.0f + e;
    if (!finite(e) || e < 0.f || !finite(denom) || denom <= 0.f) return 1;
    float sigmoid = (nonneg ? 1.0f : e) / denom;
    float silu = g * sigmoid;
    float product = silu * u;
    if (!finite(sigmoid) || !finite(silu) || !finite(product)) return 1;
    uint16_t r = narrow(product);
    if (!finite_bf16(r)) return 1;
    out[i] = r;
  }
  return 0;
}

// TP1 residual (device/qwen3-tp-batch32-kernels-v5/src/collective.rs:5-60;
// host-staged form adapters/m1-engineering-execution-v1/src/tp_execution/
// collective.rs:44-66): out = bf16((0 + partial) + residual). The reference
// rejects a nonfinite partial, a nonfinite partial sum, a nonfinite residual
// or sum, and a sum whose bf16 rounding overflows. Every element is still
// narrowed into out (the device path writes it too); rejected (may be NULL)
// receives a per-element flag, and the return value is the number of
// rejected elements (nonzero: the reference fails the batch).
uint64_t orc_residual(const float* partial, const uint16_t* residual, uint64_t count, uint16_t* out,
                      uint8_t* rejected) {
  uint64_t bad = 0;
  for (uint64_t i = 0; i < count; ++i) {
    const float p = partial[i];
    const float sum = 0.0f + p;
    const float r = widen(residual[i]);
    const float value = sum + r;
    const uint16_t rounded = narrow(value);
    out[i] = rounded;
    const bool reject = !finite(p) || !finite(sum) || !finite(r) || !finite(value) || !finite_bf16(rounded);
    if (rejected) rejected[i] = reject ? 1 : 0;
    bad += reject ? 1 : 0;
  }
  return bad;
}

// Lowest-id argmax (logits.rs:197-270; v8 FP32 logits.rs:30): strict '>' scan.
// Returns the token id, or 0xffffffff on any nonfinite value. top2_gap (may
// be NULL) receives max - (best value among the other ids), the near-tie
// measure of tools/draft_reference.py:186-197.
uint32_t orc_argmax_f32(const float* logits, uint32_t vocab, float* top2_gap) {
  if (vocab == 0 || !finite(logits[0])) return 0xffffffffu;
  uint32_t win = 0;
  float best = logits[0];
  for (uint32_t t = 1; t < vocab; ++t) {
    float c = logits[t];
    if (!finite(c)) return 0xffffffffu;
    if (c > best) {
      best = c;
      win = t;
    }
  }
  if (top2_gap) {
    float second = -INFINITY;
    for (uint32_t t = 0; t < vocab; ++t)
      if (t != win && logits[t] > second) second = logits[t];
    *top2_gap = best - second;
  }
  return win;
}

uint32_t orc_argmax_bf16(const uint16_t* logits, uint32_t vocab) {
  if (vocab == 0 || !finite_bf16(logits[0])) return 0xffffffffu;
  uint32_t win = 0;
  float best = widen(logits[0]);
  for (uint32_t t = 1; t < vocab; ++t) {
    if (!finite_bf16(logits[t])) return 0xffffffffu;
    float c = widen(logits[t]);
    if (c > best) {
      best = c;
      win = t;
    }
  }
  return win;
}

// Speculative helpers: token assembly (logits.rs:587-629) and greedy verify
// (crates/ferric-spec/src/speculation.rs:126-200).
void orc_token_assembly(const uint32_t* anchors, const uint32_t* draft, uint32_t sequences, uint32_t k,
                        uint32_t* target_ids) {
  for (uint32_t s = 0; s < sequences; ++s) {
    target_ids[(uint64_t)s * (k + 1)] = anchors[s];
    for (uint32_t i = 0; i < k; ++i) target_ids[(uint64_t)s * (k + 1) + 1 + i] = draft[(uint64_t)i * sequences + s];
  }
}

int orc_verify_greedy(const uint32_t* draft, uint32_t draft_count, const uint32_t* target, uint32_t target_count,
                      uint32_t* accepted, uint32_t* emitted, uint32_t* emitted_count) {
  if (target_count == 0) return 1;
  if (target_count != draft_count + 1) return 2;
  uint32_t a = 0;
  while (a < draft_count && draft[a] == target[a]) ++a;
  for (uint32_t i = 0; i < a; ++i) emitted[i] = draft[i];
  emitted[a] = target[a];
  *accepted = a;
  *emitted_count = a + 1;
  return 0;
}

// One sequence's compact completion record (ferric_qwen3_compact_completion_v1,
// device/qwen3-all-kernels-v1/src/logits.rs:279-520), restating the reference's
// test oracle compact_record_with_trace (device/qwen3-logits-v1/tests/reference.rs:
// 106-191). Writes 120 bytes; returns 0, or 1 where that oracle returns None.
// reads (may be NULL) receives the sequence of token reads, encoded as
// (index << 1) | is_choice, and *nreads their count (at most 2 k + 1).
int orc_compact_record(const uint32_t* choices, uint64_t nchoices, const uint32_t* draft, uint64_t ndraft,
                       uint32_t live, uint32_t slot, uint32_t generation, uint64_t epoch, const uint8_t* plan,
                       uint32_t sequences, uint32_t sequence, uint32_t active_tokens, uint32_t k, uint8_t* record,
                       uint64_t* reads, uint32_t* nreads) {
  const uint32_t kVocab = 151936;
  uint32_t nr = 0;
  auto note = [&](uint64_t index, bool choice) {
    if (reads) reads[nr] = (index << 1) | (choice ? 1u : 0u);
    ++nr;
  };
  int status = 1;
  std::memset(record, 0, 120);
  do {
    if (live == 0) {
      status = 0;
      break;
    }
    const uint32_t direct_offset = live - 1;
    bool plan_zero = true;
    for (int b = 0; b < 32; ++b) plan_zero &= plan[b] == 0;
    if (live > active_tokens || (k != 0 && live != active_tokens) || slot >= 32 || generation == 0 || plan_zero)
      break;
    const uint64_t choice_base = (uint64_t)sequence * active_tokens;
    uint32_t accepted = 0;
    bool fail = false;
    if (k != 0) {
      while (accepted < k) {
        if (accepted >= k || sequence >= sequences) { fail = true; break; }
        const uint64_t di = (uint64_t)accepted * sequences + sequence;
        note(di, false);
        if (di >= ndraft) { fail = true; break; }
        const uint32_t d = draft[di];
        if (sequence >= sequences || accepted >= active_tokens) { fail = true; break; }
        const uint64_t ti = choice_base + accepted;
        note(ti, true);
        if (ti >= nchoices) { fail = true; break; }
        const uint32_t t = choices[ti];
        if (d >= kVocab || t >= kVocab) { fail = true; break; }
        if (d != t) break;
        ++accepted;
      }
    }
    if (fail || accepted >= active_tokens) break;
    const uint64_t ci = k == 0 ? choice_base + direct_offset : choice_base + accepted;
    note(ci, true);
    if (ci >= nchoices) break;
    const uint32_t correction = choices[ci];
    if (correction >= kVocab) break;
    for (int i = 0; i < 4; ++i) record[i] = (uint8_t)(slot >> (8 * i));
    for (int i = 0; i < 4; ++i) record[4 + i] = (uint8_t)(generation >> (8 * i));
    for (int i = 0; i < 8; ++i) record[8 + i] = (uint8_t)(epoch >> (8 * i));
    std::memcpy(record + 16, plan, 32);
    record[48] = (uint8_t)accepted;
    record[49] = (uint8_t)(accepted + 1);
    for (uint32_t t = 0; t < accepted; ++t) {
      const uint32_t v = draft[(uint64_t)t * sequences + sequence];
      for (int i = 0; i < 4; ++i) record[52 + 4 * t + i] = (uint8_t)(v >> (8 * i));
    }
    for (int i = 0; i < 4; ++i) record[52 + 4 * accepted + i] = (uint8_t)(correction >> (8 * i));
    status = 0;
  } while (false);
  if (status) std::memset(record, 0, 120);
  if (nreads) *nreads = nr;
  return status;
}

// ---- synthetic inputs (ferric_synth.h) ----
void orc_synth_fill(uint16_t* dst, uint64_t count, uint64_t tensor_seed, float scale) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)count; ++i) dst[i] = fh_synth_bf16(tensor_seed, (uint64_t)i, scale);
}

uint64_t orc_splitmix64(uint64_t x) { return fh_splitmix64(x); }

uint64_t orc_synth_tensor_seed(uint64_t seed, uint32_t kind, uint32_t layer) {
  return fh_synth_tensor_seed(seed, kind, layer);
}

float orc_synth_scale(double sigma) { return fh_synth_scale(sigma); }

// Threads the OpenMP regions above will use (the CPU baseline's core count).
int orc_threads(void) { return omp_get_max_threads(); }

}  // extern "C"

// ---- whole-model forward step -------------------------------------------------
// The op order of EngineeringTpBatchExecutionV2::forward
// (tp_execution/batched.rs:1746-2454) and of ferric-spec's layer graph
// (crates/ferric-spec/src/graph.rs:961-1010): embedding; per layer input
// RMSNorm -> Q, K, V -> Q-norm, K-norm (width 128) -> RoPE -> KV append (K
// rotated, V raw) -> attention -> O + residual -> post RMSNorm -> gate, up ->
// SwiGLU -> down + residual; final RMSNorm -> FP32 LM head -> argmax.

struct OrcModel {
  uint32_t layers, hidden, qh, kvh, inter, vocab, tied, theta;
  float eps;
  // 0: serial (v1) sums; 1: the wave-order profiles; 2: the wave order with
  // a planted mistake (the gate and up projections narrowed to bf16 by
  // truncation instead of round-to-nearest-even: a 1-ulp-biased rounding in
  // one GEMM, which tests use to show that the drift bound between the two
  // legal orders catches such a bug).
  int order = 0;
  // row-major bf16 weights, indexed by tensor kind (ferric_hip.h order)
  std::vector<uint16_t> head, embed, final_norm;
  struct Layer {
    std::vector<uint16_t> in_norm, post_norm, q_norm, k_norm, wq, wk, wv, wo, wg, wu, wd;
  };
  std::vector<Layer> L;
  // KV pool: [layer][2][pages][16][kvh][128]
  uint32_t pages = 0;
  std::vector<uint16_t> kv;
  uint64_t slab() const { return (uint64_t)pages * 16 * kvh * 128; }
  uint16_t* cache(uint32_t layer, uint32_t which) { return kv.data() + ((uint64_t)layer * 2 + which) * slab(); }
};

extern "C" {

OrcModel* orc_model_create(uint32_t layers, uint32_t hidden, uint32_t qh, uint32_t kvh, uint32_t inter,
                           uint32_t vocab, uint32_t tied, uint32_t theta, float eps, uint32_t pages) {
  OrcModel* m = new OrcModel();
  m->layers = layers;
  m->hidden = hidden;
  m->qh = qh;
  m->kvh = kvh;
  m->inter = inter;
  m->vocab = vocab;
  m->tied = tied;
  m->theta = theta;
  m->eps = eps;
  m->L.resize(layers);
  m->pages = pages;
  m->kv.assign(m->slab() * 2 * layers, 0);
  return m;
}

void orc_model_destroy(OrcModel* m) { delete m; }

// Reduction order of the model's later steps: 0 serial (v1), 1 wave profiles,
// 2 wave profiles with the planted gate/up truncation (tests only).
void orc_model_set_order(OrcModel* m, int order) { m->order = order; }

// Pointer to a weight's row-major storage, resized on first use.
uint16_t* orc_model_weight(OrcModel* m, uint32_t kind, uint32_t layer, uint64_t elements) {
  std::vector<uint16_t>* v = nullptr;
  switch (kind) {
    case 0: v = &m->head; break;
    case 1: v = &m->embed; break;
    case 2: v = &m->final_norm; break;
    case 3: v = &m->L[layer].in_norm; break;
    case 4: v = &m->L[layer].post_norm; break;
    case 5: v = &m->L[layer].q_norm; break;
    case 6: v = &m->L[layer].k_norm; break;
    case 7: v = &m->L[layer].wq; break;
    case 8: v = &m->L[layer].wk; break;
    case 9: v = &m->L[layer].wv; break;
    case 10: v = &m->L[layer].wo; break;
    case 11: v = &m->L[layer].wg; break;
    case 12: v = &m->L[layer].wu; break;
    case 13: v = &m->L[layer].wd; break;
    default: return nullptr;
  }
  if (v->size() != elements) v->assign(elements, 0);
  return v->data();
}

// Same tensors, seeds and values as fh_synthesize_weights.
void orc_model_synthesize(OrcModel* m, uint64_t seed, float sigma) {
  const float scale = fh_synth_scale(sigma);
  const uint64_t H = m->hidden, Q = (uint64_t)m->qh * 128, KV = (uint64_t)m->kvh * 128, I = m->inter, V = m->vocab;
  auto gen = [&](uint32_t kind, uint32_t layer, uint64_t count, bool norm) {
    uint16_t* p = orc_model_weight(m, kind, layer, count);
    if (norm)
      std::fill(p, p + count, (uint16_t)0x3f80);
    else
      orc_synth_fill(p, count, fh_synth_tensor_seed(seed, kind, layer), scale);
  };
  const uint32_t nl = 0xffffffffu;
  if (!m->tied) gen(0, nl, V * H, false);
  gen(1, nl, V * H, false);
  gen(2, nl, H, true);
  for (uint32_t l = 0; l < m->layers; ++l) {
    gen(3, l, H, true);
    gen(4, l, H, true);
    gen(5, l, 128, true);
    gen(6, l, 128, true);
    gen(7, l, Q * H, false);
    gen(8, l, KV * H, false);
    gen(9, l, KV * H, false);
    gen(10, l, H * Q, false);
    gen(11, l, I * H, false);
    gen(12, l, I * H, false);
    gen(13, l, H * I, false);
  }
}

uint16_t* orc_model_kv(OrcModel* m, uint32_t layer, uint32_t which) { return m->cache(layer, which); }

// Same values as fh_kv_fill_synthetic: positions [0, lengths[i]) of row i.
void orc_model_kv_fill(OrcModel* m, uint64_t seed, float sigma, const uint32_t* tables, uint32_t stride,
                       const uint32_t* lengths, const uint64_t* keys, uint32_t rows, uint32_t context_stride) {
  const float scale = fh_synth_scale(sigma);
  const uint64_t re = (uint64_t)m->kvh * 128;
  for (uint32_t l = 0; l < m->layers; ++l)
    for (uint32_t w = 0; w < 2; ++w) {
      const uint64_t ts = fh_synth_tensor_seed(seed, FH_SYNTH_KIND_KV_KEY + w, l);
      uint16_t* c = m->cache(l, w);
      for (uint32_t r = 0; r < rows; ++r) {
#pragma omp parallel for schedule(static)
        for (int64_t p = 0; p < (int64_t)lengths[r]; ++p) {
          const uint32_t page = tables[(uint64_t)r * stride + p / 16];
          const uint64_t dst = ((uint64_t)page * 16 + (p % 16)) * re;
          const uint64_t idx = (keys[r] * context_stride + (uint64_t)p) * re;
          for (uint64_t e = 0; e < re; ++e) c[dst + e] = fh_synth_bf16(ts, idx + e, scale);
        }
      }
    }
}

// One decoder layer in place on h[rows][hidden], writing K/V to kc/vc.
// Returns 0, or 1 where the reference would trap.
// The model's projections and width-H norms in its reduction order (QK-norm
// keeps the serial width-128 sum in both orders).
static void model_gemm(OrcModel* m, const uint16_t* a, const uint16_t* b, uint32_t rows, uint32_t n, uint32_t k,
                       uint16_t* out, float* out_f32, bool planted = false) {
  if (m->order == 2 && planted && out) {
    std::vector<float> f((uint64_t)rows * n);
    orc_gemm_wave(a, b, rows, n, k, nullptr, f.data());
    for (uint64_t i = 0; i < f.size(); ++i) out[i] = (uint16_t)(bits_of(f[i]) >> 16);  // truncation
  } else if (m->order >= 1) {
    orc_gemm_wave(a, b, rows, n, k, out, out_f32);
  } else {
    orc_gemm(a, b, nullptr, rows, n, k, 0, out, out_f32);
  }
}

static int model_norm(OrcModel* m, const uint16_t* x, const uint16_t* w, uint32_t rows, uint32_t width,
                      uint16_t* out) {
  if (m->order == 3) return orc_rmsnorm_exact(x, w, rows, width, m->eps, out);
  if (m->order >= 1) return orc_rmsnorm_wave(x, w, rows, width, m->eps, out);
  return orc_rmsnorm(x, nullptr, w, rows, width, m->eps, 0, nullptr, out);
}

static int run_layer(OrcModel* m, uint32_t l, uint16_t* h, uint32_t rows, const uint32_t* positions,
                     const uint32_t* tables, const uint32_t* page_counts, uint32_t stride, const float* cosr,
                     const float* sinr, uint16_t* kc, uint16_t* vc) {
  const uint32_t H = m->hidden, QH = m->qh, KVH = m->kvh, Q = QH * 128, KV = KVH * 128, I = m->inter;
  std::vector<uint16_t> xn((uint64_t)rows * H), q((uint64_t)rows * Q), k((uint64_t)rows * KV),
      v((uint64_t)rows * KV), qn((uint64_t)rows * Q), kn((uint64_t)rows * KV), qr((uint64_t)rows * Q),
      kr((uint64_t)rows * KV), attn((uint64_t)rows * Q), gate((uint64_t)rows * I), up((uint64_t)rows * I),
      act((uint64_t)rows * I);
  OrcModel::Layer& W = m->L[l];
  if (model_norm(m, h, W.in_norm.data(), rows, H, xn.data())) return 1;
  model_gemm(m, xn.data(), W.wq.data(), rows, Q, H, q.data(), nullptr);
  model_gemm(m, xn.data(), W.wk.data(), rows, KV, H, k.data(), nullptr);
  model_gemm(m, xn.data(), W.wv.data(), rows, KV, H, v.data(), nullptr);
  if (orc_rmsnorm(q.data(), nullptr, W.q_norm.data(), rows * QH, 128, m->eps, 0, nullptr, qn.data())) return 1;
  if (orc_rmsnorm(k.data(), nullptr, W.k_norm.data(), rows * KVH, 128, m->eps, 0, nullptr, kn.data())) return 1;
  for (uint32_t r = 0; r < rows; ++r) {
    for (uint32_t hh = 0; hh < QH; ++hh)
      for (uint32_t i = 0; i < 64; ++i) {
        uint16_t o[2];
        const uint64_t b = (uint64_t)r * Q + hh * 128;
        orc_rope_pair(qn[b + i], qn[b + i + 64], cosr[r * 64ull + i], sinr[r * 64ull + i], o);
        qr[b + i] = o[0];
        qr[b + i + 64] = o[1];
      }
    for (uint32_t hh = 0; hh < KVH; ++hh)
      for (uint32_t i = 0; i < 64; ++i) {
        uint16_t o[2];
        const uint64_t b = (uint64_t)r * KV + hh * 128;
        orc_rope_pair(kn[b + i], kn[b + i + 64], cosr[r * 64ull + i], sinr[r * 64ull + i], o);
        kr[b + i] = o[0];
        kr[b + i + 64] = o[1];
      }
  }
  for (uint64_t i = 0; i < (uint64_t)rows * Q; ++i)
    if (!finite_bf16(qr[i])) return 1;
  // KV append: every row before any attention (batched.rs:1995-2035).
  for (uint32_t r = 0; r < rows; ++r) {
    const uint32_t pos = positions[r], lp = pos / 16;
    if (lp >= page_counts[r]) return 1;
    const uint32_t page = tables[(uint64_t)r * stride + lp];
    if (page >= m->pages) return 1;
    const uint64_t dst = orc_cache_index(page, pos % 16, KVH, 0, 0);
    std::memcpy(kc + dst, kr.data() + (uint64_t)r * KV, (uint64_t)KV * 2);
    std::memcpy(vc + dst, v.data() + (uint64_t)r * KV, (uint64_t)KV * 2);
  }
  int bad = 0;
#pragma omp parallel for collapse(2) schedule(dynamic) reduction(| : bad)
  for (int64_t r = 0; r < (int64_t)rows; ++r)
    for (int64_t hh = 0; hh < (int64_t)QH; ++hh) {
      const uint32_t kvhead = (uint32_t)hh / (QH / KVH);
      bad |= attention_head_ordered(qr.data() + (uint64_t)r * Q + hh * 128, kc, vc, tables + (uint64_t)r * stride,
                                    page_counts[r], m->pages, positions[r], KVH, kvhead,
                                    attn.data() + (uint64_t)r * Q + hh * 128, m->order >= 1 ? 1 : 0);
    }
  if (bad) return 1;
  // O projection: FP32 partial, then the TP1 residual.
  {
    std::vector<float> part((uint64_t)rows * H);
    model_gemm(m, attn.data(), W.wo.data(), rows, H, Q, nullptr, part.data());
    if (orc_residual(part.data(), h, (uint64_t)rows * H, h, nullptr)) return 1;
  }
  if (model_norm(m, h, W.post_norm.data(), rows, H, xn.data())) return 1;
  model_gemm(m, xn.data(), W.wg.data(), rows, I, H, gate.data(), nullptr, true);
  model_gemm(m, xn.data(), W.wu.data(), rows, I, H, up.data(), nullptr, true);
  if (orc_swiglu(gate.data(), up.data(), (uint64_t)rows * I, act.data())) return 1;
  {
    std::vector<float> part((uint64_t)rows * H);
    model_gemm(m, act.data(), W.wd.data(), rows, H, I, nullptr, part.data());
    if (orc_residual(part.data(), h, (uint64_t)rows * H, h, nullptr)) return 1;
  }
  return 0;
}

// One forward step over `rows` token rows. tables: [rows][stride] page
// lists (page_counts[r] valid entries). Writes choices[rows]; optional
// logits [rows][vocab] (FP32), hidden [layers][rows][hidden] (residual stream
// after each layer) and gaps [rows] (top-2 gap). Returns 0, or 1 + the layer
// index where the reference would trap (nonfinite / bad index). seconds (may
// be NULL) receives the wall time of [all layers, embedding + final norm +
// head + argmax].
int orc_model_forward(OrcModel* m, const uint32_t* tokens, const uint32_t* positions, const uint32_t* tables,
                      const uint32_t* page_counts, uint32_t stride, uint32_t rows, uint32_t* choices, float* logits,
                      uint16_t* hidden_capture, float* gaps, double* seconds) {
  const uint32_t H = m->hidden, V = m->vocab;
  const double t_begin = omp_get_wtime();
  double t_layers_begin = 0.0, t_layers_end = 0.0;
  std::vector<uint16_t> h((uint64_t)rows * H), xn((uint64_t)rows * H);
  if (orc_embedding(tokens, m->embed.data(), rows, H, V, h.data())) return 1;
  std::vector<float> cosr((uint64_t)rows * 64), sinr((uint64_t)rows * 64);
  for (uint32_t r = 0; r < rows; ++r) orc_rope_table(positions[r], m->theta, &cosr[r * 64ull], &sinr[r * 64ull]);
  t_layers_begin = omp_get_wtime();
  for (uint32_t l = 0; l < m->layers; ++l) {
    if (run_layer(m, l, h.data(), rows, positions, tables, page_counts, stride, cosr.data(), sinr.data(),
                  m->cache(l, 0), m->cache(l, 1)))
      return 1 + (int)l;
    if (hidden_capture) std::memcpy(hidden_capture + (uint64_t)l * rows * H, h.data(), (uint64_t)rows * H * 2);
  }
  t_layers_end = omp_get_wtime();
  const int fail = 1 + (int)m->layers;
  if (model_norm(m, h.data(), m->final_norm.data(), rows, H, xn.data())) return fail;
  std::vector<float> lg((uint64_t)rows * V);
  model_gemm(m, xn.data(), m->tied ? m->embed.data() : m->head.data(), rows, V, H, nullptr, lg.data());
  for (uint32_t r = 0; r < rows; ++r) {
    float gap = 0.f;
    uint32_t c = orc_argmax_f32(lg.data() + (uint64_t)r * V, V, &gap);
    if (c == 0xffffffffu) return fail;
    choices[r] = c;
    if (gaps) gaps[r] = gap;
  }
  if (logits) std::memcpy(logits, lg.data(), lg.size() * 4);
  if (seconds) {
    const double t_end = omp_get_wtime();
    seconds[0] = t_layers_end - t_layers_begin;
    seconds[1] = (t_end - t_begin) - seconds[0];
  }
  return 0;
}


// Final RMSNorm + FP32 LM head + argmax from a caller-given residual stream
// hidden_in [rows][hidden] (the head's own error on the GPU's final hidden
// state). Returns 0, or 1 where the reference traps.
int orc_model_head(OrcModel* m, const uint16_t* hidden_in, uint32_t rows, float* logits, uint32_t* choices,
                   float* gaps) {
  const uint32_t H = m->hidden, V = m->vocab;
  std::vector<uint16_t> xn((uint64_t)rows * H);
  if (model_norm(m, hidden_in, m->final_norm.data(), rows, H, xn.data())) return 1;
  model_gemm(m, xn.data(), m->tied ? m->embed.data() : m->head.data(), rows, V, H, nullptr, logits);
  for (uint32_t r = 0; r < rows; ++r) {
    float gap = 0.f;
    const uint32_t c = orc_argmax_f32(logits + (uint64_t)r * V, V, &gap);
    if (c == 0xffffffffu) return 1;
    choices[r] = c;
    if (gaps) gaps[r] = gap;
  }
  return 0;
}

// Layer `layer` alone, from a caller-given input residual stream hidden_in
// [rows][hidden] to hidden_out, against a scratch copy of that layer's KV
// (the model's pool is left untouched). Used to measure one layer's numerical
// error on the GPU's own input. Returns 0, or 1 where the reference traps.
// kc_in / vc_in (may be NULL): the layer's K and V pools to start from
// instead of the model's own (e.g. another implementation's KV history, so
// that only the layer's own arithmetic differs).
int orc_model_layer_isolated(OrcModel* m, uint32_t layer, const uint16_t* hidden_in, const uint32_t* positions,
                             const uint32_t* tables, const uint32_t* page_counts, uint32_t stride, uint32_t rows,
                             const uint16_t* kc_in, const uint16_t* vc_in, uint16_t* hidden_out) {
  const uint64_t n = (uint64_t)rows * m->hidden;
  std::memcpy(hidden_out, hidden_in, n * 2);
  const uint16_t* k0 = kc_in ? kc_in : m->cache(layer, 0);
  const uint16_t* v0 = vc_in ? vc_in : m->cache(layer, 1);
  std::vector<uint16_t> kc(k0, k0 + m->slab());
  std::vector<uint16_t> vc(v0, v0 + m->slab());
  std::vector<float> cosr((uint64_t)rows * 64), sinr((uint64_t)rows * 64);
  for (uint32_t r = 0; r < rows; ++r) orc_rope_table(positions[r], m->theta, &cosr[r * 64ull], &sinr[r * 64ull]);
  return run_layer(m, layer, hidden_out, rows, positions, tables, page_counts, stride, cosr.data(), sinr.data(),
                   kc.data(), vc.data());
}

}  // extern "C"
