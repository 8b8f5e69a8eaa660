// QK-norm + RoPE + paged KV append of one (row, head) of a bf16 QKV row,
// computed by one lane (the prefill path: the lane-per-head kernel in
// k_norm.hip, and the QKV projection's fused epilogue in k_gemm_large.hip,
// which stages its output rows in LDS and calls this on them).
//
// Reference semantics: qwen3_rmsnorm_v1 at width 128 per head
// (device/qwen3-all-kernels-v1/src/rmsnorm.rs:380-526; the serial sum of
// squares of rmsnorm.rs:421-438, each square rounded before the add),
// qwen3_rope_v1 (rope_kv.rs:102: a' = a c - b s, b' = b c + a s on pairs
// (i, i + 64)), and qwen3_paged_kv_write_v1 (rope_kv.rs:261-388: K rotated,
// V raw, slot pages[pos / 16] * 16 + pos % 16).
#pragma once

#include "common.hpp"

namespace fh {

typedef unsigned int qk_u32x4 __attribute__((ext_vector_type(4)));

// Correctly rounded square root of a positive normal float. The hardware
// square root (v_sqrt_f32, what __fsqrt_rn becomes on this target) is only
// within 1 ulp, so one correction step picks among its estimate s and the
// neighbours s- and s+: the root rounds down to s- exactly when
// x <= s- * s, and up to s+ exactly when x > s+ * s (both products exact
// inside the FMA). A float x and either product differ by a multiple of
// ulp(s)^2, while these thresholds sit within ulp(s)^2 / 4 of the true
// rounding midpoints, so the comparisons decide exactly as the midpoints
// would. Below 2^-64 those differences would underflow, so x is first
// scaled by 2^64 and the root by 2^-32 (both exact). Checked against the
// midpoint definition for every positive normal float.
__device__ __forceinline__ float sqrt_rn(float x) {
  const bool tiny = x < 0x1p-64f;
  const float xs = tiny ? x * 0x1p64f : x;
  const float s = __builtin_amdgcn_sqrtf(xs);
  const uint32_t u = __builtin_bit_cast(uint32_t, s);
  const float down = __builtin_bit_cast(float, u - 1u), up = __builtin_bit_cast(float, u + 1u);
  float r = s;
  if (__builtin_fmaf(-down, s, xs) <= 0.0f) r = down;
  if (__builtin_fmaf(-up, s, xs) > 0.0f) r = up;
  return tiny ? r * 0x1p-32f : r;
}

// Inverse RMS exactly as qwen3_rmsnorm_v1 forms it
// (device/qwen3-all-kernels-v1/src/rmsnorm.rs:440-456): mean = sum / width
// (a division), + epsilon, correctly rounded sqrt, then 1 / sqrt.
__device__ __forceinline__ float inverse_rms(float sum, float width, float eps) {
  float mean_square = __fdiv_rn(sum, width);
  float stabilized = mean_square + eps;
  float denominator = sqrt_rn(stabilized);
  return __fdiv_rn(1.0f, denominator);
}

// Normalize-then-round, weight, round again (rmsnorm.rs:486-503; the witness
// in device/qwen3-rmsnorm-v1/tests/reference.rs:264-274 pins the double round).
__device__ __forceinline__ uint32_t norm_weight_bf16(float x, float inv, float w) {
  float normalized = round_bf16(x * inv);
  return f32_to_bf16(normalized * w);
}

// The same with the narrowing as integer operations (equal results). The
// lane-per-head routine below uses it: with the conversion instruction there
// the compiler hoists every cos/sin and weight load to the top and spills.
__device__ __forceinline__ uint32_t norm_weight_bf16_int(float x, float inv, float w) {
  float normalized = bf16_to_f32(f32_to_bf16_int(x * inv));
  return f32_to_bf16_int(normalized * w);
}

// QK-norm + RoPE of one normalized head held by a wave: lane l holds
// elements l (a) and l + 64 (b) as bf16-valued floats, wa/wb the norm
// weights of those elements, c/s the RoPE factors of pair l at the row's
// position. The square sum runs serially in element order 0..127 (one
// rounding per square and per add, rmsnorm.rs:421-438) through lane reads.
// ra/rb: the rotated bf16 outputs of elements l and l + 64. Returns true
// when a value or the sum is nonfinite. The decode QK-norm kernel and the
// decode attention kernel's fused form both call this, so their outputs are
// bit-identical.
// The part after the square sum, given it (the block attention forms the
// sums of its heads another way, in the same order).
__device__ __forceinline__ bool qknorm_rope_wave_head_from_sum(float a, float b, float sum, float wa, float wb,
                                                               float c, float s, float eps, uint32_t& ra,
                                                               uint32_t& rb) {
  bool bad = !is_finite_f32(a) | !is_finite_f32(b);
  const float inv = inverse_rms(sum, 128.0f, eps);
  bad |= !is_finite_f32(sum) | !is_finite_f32(inv);
  const float an = bf16_to_f32(norm_weight_bf16(a, inv, wa));
  const float bn = bf16_to_f32(norm_weight_bf16(b, inv, wb));
  const float a_cos = an * c, b_sin = bn * s, b_cos = bn * c, a_sin = an * s;
  ra = f32_to_bf16(a_cos - b_sin);
  rb = f32_to_bf16(b_cos + a_sin);
  bad |= ((ra & 0x7f80u) == 0x7f80u) | ((rb & 0x7f80u) == 0x7f80u);
  return bad;
}

__device__ __forceinline__ bool qknorm_rope_wave_head(float a, float b, float wa, float wb, float c, float s,
                                                      float eps, uint32_t& ra, uint32_t& rb) {
  const float sqa = a * a, sqb = b * b;
  float sum = 0.f;
#pragma unroll
  for (int l = 0; l < 64; ++l) sum = sum + lane_bcast(sqa, l);
#pragma unroll
  for (int l = 0; l < 64; ++l) sum = sum + lane_bcast(sqb, l);
  return qknorm_rope_wave_head_from_sum(a, b, sum, wa, wb, c, s, eps, ra, rb);
}

struct QkvRopeArgs {
  const uint16_t* q_norm;
  const uint16_t* k_norm;
  const float* cos_t;  // [context][64]
  const float* sin_t;
  const uint32_t* positions;
  const uint32_t* table;  // [rows][stride]
  uint16_t* q_out;        // [rows][qh][128]
  uint16_t* k_cache;      // [pages][16][kvh][128]
  uint16_t* v_cache;
  uint32_t qh, kvh, stride, pages, context;
  float eps;
  uint32_t* err;
};

// A row's position and KV slot (slot_ok false: position or page outside the
// envelope; nothing is written to the cache then, and head 0 reports it).
struct QkvRowSlot {
  uint32_t pos, slot;
  bool slot_ok;
};

__device__ __forceinline__ QkvRowSlot qkv_row_slot(uint32_t row, const QkvRopeArgs& a) {
  QkvRowSlot r{a.positions[row], 0u, false};
  r.slot_ok = r.pos < a.context && r.pos / 16 < a.stride;
  if (r.slot_ok) {
    const uint32_t page = a.table[(uint64_t)row * a.stride + r.pos / 16];
    r.slot_ok = page < a.pages;
    r.slot = (page * 16u + (r.pos & 15u)) * a.kvh;
  }
  return r;
}

// src: the head's 128 bf16 values (16-byte aligned, global or LDS). Query
// heads 0 .. qh - 1 go to q_out, key heads qh .. qh + kvh - 1 (normed and
// rotated) and value heads (raw) to the row's KV slot. kHoist: cos/sin pairs
// requested at a time (8 keeps the lane-per-head kernel's registers low
// enough for its occupancy; a caller with few waves takes all 32 at once).
// kHwCvt: narrow with the conversion instruction (equal results, far fewer
// instructions) where the caller has the registers for it.
template <int kHoist = 8, bool kHwCvt = false>
__device__ __forceinline__ void qknorm_rope_kv_head(const qk_u32x4* src, uint32_t row, uint32_t head,
                                                    const QkvRopeArgs& a, const QkvRowSlot rs) {
  uint32_t x[64];  // x[i] = elements 2 i (low half) and 2 i + 1 (high half)
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const qk_u32x4 v = src[i];
    x[4 * i] = v[0];
    x[4 * i + 1] = v[1];
    x[4 * i + 2] = v[2];
    x[4 * i + 3] = v[3];
  }
  const uint32_t pos = rs.pos, slot = rs.slot;
  const bool slot_ok = rs.slot_ok;
  if (!slot_ok && head == 0) raise_error(a.err, ERR_PAGE);
  const uint32_t heads = a.qh + a.kvh;
  if (head >= heads) {
    if (slot_ok) {
      qk_u32x4* vo = reinterpret_cast<qk_u32x4*>(a.v_cache + ((uint64_t)slot + (head - heads)) * 128);
#pragma unroll
      for (int i = 0; i < 16; ++i) vo[i] = qk_u32x4{x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]};
    }
    return;
  }
  // (A nonfinite element makes the sum nonfinite, which is checked.)
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    const float e0 = lo_bf16(x[i]), e1 = hi_bf16(x[i]);
    const float s0 = e0 * e0, s1 = e1 * e1;
    sum = sum + s0;
    sum = sum + s1;
  }
  const float inv = inverse_rms(sum, 128.0f, a.eps);
  bool bad = !is_finite_f32(sum) | !is_finite_f32(inv);
  // Keep only the packed words live across the reduction (the unpacked
  // values are recomputed), or the lane runs out of registers.
#pragma unroll
  for (int i = 0; i < 64; ++i) asm volatile("" : "+v"(x[i]));
  // Normalized in place, then rotated in place (pair words i and i + 32
  // hold elements 2 i, 2 i + 1 and 2 i + 64, 2 i + 65).
  const qk_u32x4* wn = reinterpret_cast<const qk_u32x4*>(head < a.qh ? a.q_norm : a.k_norm);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const qk_u32x4 w = wn[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t xi = x[4 * i + j];
      const uint32_t lo = kHwCvt ? norm_weight_bf16(lo_bf16(xi), inv, lo_bf16(w[j]))
                                 : norm_weight_bf16_int(lo_bf16(xi), inv, lo_bf16(w[j]));
      const uint32_t hi = kHwCvt ? norm_weight_bf16(hi_bf16(xi), inv, hi_bf16(w[j]))
                                 : norm_weight_bf16_int(hi_bf16(xi), inv, hi_bf16(w[j]));
      x[4 * i + j] = lo | (hi << 16);
    }
  }
  const float* ct = a.cos_t + (uint64_t)(pos < a.context ? pos : 0) * 64;
  const float* st = a.sin_t + (uint64_t)(pos < a.context ? pos : 0) * 64;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    if (i % kHoist == 0) __builtin_amdgcn_sched_barrier(0);  // bounds how many cos/sin loads are hoisted
    const float2 c = *reinterpret_cast<const float2*>(ct + 2 * i);
    const float2 sn = *reinterpret_cast<const float2*>(st + 2 * i);
    const float a0 = lo_bf16(x[i]), a1 = hi_bf16(x[i]);
    const float b0 = lo_bf16(x[i + 32]), b1 = hi_bf16(x[i + 32]);
    const float a0c = a0 * c.x, b0s = b0 * sn.x, b0c = b0 * c.x, a0s = a0 * sn.x;
    const float a1c = a1 * c.y, b1s = b1 * sn.y, b1c = b1 * c.y, a1s = a1 * sn.y;
    const uint32_t ra0 = kHwCvt ? f32_to_bf16(a0c - b0s) : f32_to_bf16_int(a0c - b0s);
    const uint32_t rb0 = kHwCvt ? f32_to_bf16(b0c + a0s) : f32_to_bf16_int(b0c + a0s);
    const uint32_t ra1 = kHwCvt ? f32_to_bf16(a1c - b1s) : f32_to_bf16_int(a1c - b1s);
    const uint32_t rb1 = kHwCvt ? f32_to_bf16(b1c + a1s) : f32_to_bf16_int(b1c + a1s);
    bad |= ((ra0 & 0x7f80u) == 0x7f80u) | ((rb0 & 0x7f80u) == 0x7f80u) | ((ra1 & 0x7f80u) == 0x7f80u) |
           ((rb1 & 0x7f80u) == 0x7f80u);
    x[i] = ra0 | (ra1 << 16);
    x[i + 32] = rb0 | (rb1 << 16);
  }
  qk_u32x4* dst = nullptr;
  if (head < a.qh)
    dst = reinterpret_cast<qk_u32x4*>(a.q_out + ((uint64_t)row * a.qh + head) * 128);
  else if (slot_ok)
    dst = reinterpret_cast<qk_u32x4*>(a.k_cache + ((uint64_t)slot + (head - a.qh)) * 128);
  if (dst) {
#pragma unroll
    for (int i = 0; i < 16; ++i) dst[i] = qk_u32x4{x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]};
  }
  if (bad) raise_error(a.err, ERR_NONFINITE);
}

}  // namespace fh
