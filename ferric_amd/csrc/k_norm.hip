// K2 RMSNorm (wavefront reduction), K3 QK-norm + RoPE + paged KV append
// (one launch per layer), and the standalone K6 SwiGLU.
#include "common.hpp"
#include "kernels.hpp"

namespace fh {

namespace {

constexpr int kNormThreads = 256;

__device__ __forceinline__ float block_sum_ordered(float v, float* red) {
  // Wave butterfly, then the four wave totals added in wave order.
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int w = 1; w < kNormThreads / 64; ++w) t += red[w];
  return t;
}

// Inverse RMS exactly as qwen3_rmsnorm_v1 forms it
// (device/qwen3-all-kernels-v1/src/rmsnorm.rs:440-456): mean = sum / width
// (a division), + epsilon, correctly rounded sqrt, then 1 / sqrt.
__device__ __forceinline__ float inverse_rms(float sum, float width, float eps) {
  float mean_square = sum / width;
  float stabilized = mean_square + eps;
  float denominator = __fsqrt_rn(stabilized);
  return __fdiv_rn(1.0f, denominator);
}

// Normalize-then-round, weight, round again (rmsnorm.rs:486-503; the witness
// in device/qwen3-rmsnorm-v1/tests/reference.rs:264-274 pins the double round).
__device__ __forceinline__ uint32_t norm_weight_bf16(float x, float inv, float w) {
  float normalized = round_bf16(x * inv);
  return f32_to_bf16(normalized * w);
}

// One workgroup per row; each thread owns 16-byte chunks c = tid, tid + 256, ...
// Width 1024 or 4096 (up to 8192). Squares are summed per thread in ascending
// chunk order, then by the ordered block reduction above. This reassociates
// the reference's serial sum (rmsnorm.rs:421-438), as the reference's own
// wave variant does (device/qwen3-tp-wave-rmsnorm-kernels-v15/src/rmsnorm.rs:20).
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ w,
                                                               uint16_t* __restrict__ y, uint32_t width, float eps,
                                                               uint32_t* err) {
  __shared__ float red[kNormThreads / 64];
  const uint32_t row = blockIdx.x;
  const uint16_t* xr = x + (uint64_t)row * width;
  const uint32_t chunks = width / 8;
  constexpr int kMaxPerThread = 4;  // width <= 8192
  uint4 v[kMaxPerThread];
  float sum = 0.f;
  bool bad = false;
#pragma unroll
  for (int j = 0; j < kMaxPerThread; ++j) {
    uint32_t c = threadIdx.x + j * kNormThreads;
    if (c < chunks) {
      v[j] = *reinterpret_cast<const uint4*>(xr + c * 8);
      uint32_t words[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float a = lo_bf16(words[q]), b = hi_bf16(words[q]);
        bad |= !is_finite_f32(a) | !is_finite_f32(b);
        sum = sum + a * a;
        sum = sum + b * b;
      }
    }
  }
  float total = block_sum_ordered(sum, red);
  float inv = inverse_rms(total, (float)width, eps);
  if (!is_finite_f32(total) || !is_finite_f32(inv)) bad = true;
  uint16_t* yr = y + (uint64_t)row * width;
#pragma unroll
  for (int j = 0; j < kMaxPerThread; ++j) {
    uint32_t c = threadIdx.x + j * kNormThreads;
    if (c < chunks) {
      uint4 wv = *reinterpret_cast<const uint4*>(w + c * 8);
      uint32_t xs[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
      uint32_t ws[4] = {wv.x, wv.y, wv.z, wv.w};
      uint32_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t a = norm_weight_bf16(lo_bf16(xs[q]), inv, lo_bf16(ws[q]));
        uint32_t b = norm_weight_bf16(hi_bf16(xs[q]), inv, hi_bf16(ws[q]));
        bad |= ((a & 0x7f80u) == 0x7f80u) | ((b & 0x7f80u) == 0x7f80u);
        o[q] = a | (b << 16);
      }
      *reinterpret_cast<uint4*>(yr + c * 8) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
  if (bad) raise_error(err, ERR_NONFINITE);
}

// Per-row QK-norm over the 128-wide heads, split-half RoPE, and the paged KV
// append, fused. One workgroup per token row:
//  1. the row's q and k heads are staged in LDS as f32;
//  2. thread h < heads sums its head's squares serially in ascending order,
//     which is exactly qwen3_rmsnorm_v1 at width 128 (rmsnorm.rs:421-438, as
//     called for QK-norm at tp_execution/batched.rs:1956-1982);
//  3. every (head, pair) computes bf16(bf16(x*inv)*w) for both halves, then
//     the RoPE pair with separately rounded products (rope_kv.rs:102-240,
//     v5 rope_kv.rs:60-80): a' = a*c - b*s, b' = b*c + a*s, each narrowed once;
//  4. rotated k and raw v go to cache[(page*16 + pos%16)][kv_head][128], the
//     slot of qwen3_paged_kv_write_v1 (rope_kv.rs:261-388).
__global__ __launch_bounds__(kNormThreads) void qknorm_rope_kv_kernel(
    const uint16_t* __restrict__ qkv, const float* __restrict__ qkv_part, uint32_t splits,
    const uint16_t* __restrict__ q_norm, const uint16_t* __restrict__ k_norm, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, const uint32_t* __restrict__ positions, const uint32_t* __restrict__ table,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache, uint32_t qh,
    uint32_t kvh, uint32_t stride, uint32_t pages, uint32_t context, float eps, uint32_t* err) {
  extern __shared__ float smem[];
  const uint32_t heads = qh + kvh;            // heads that are normalized and rotated
  const uint32_t all_heads = qh + 2 * kvh;    // plus the V heads
  float* xs = smem;                           // [all_heads][129] (padded against bank conflicts)
  float* inv_s = smem + all_heads * 129;      // [heads]
  const uint32_t row = blockIdx.x;
  const uint32_t ld = all_heads * 128;

  // Projection outputs of this row, as bf16 values: either the bf16 row, or
  // bf16(P_0 + P_1 + ...) over the split-K slabs (one rounding, as the
  // reference's one RNE per projection output).
  if (splits == 0) {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(qkv + (uint64_t)row * ld);
    for (uint32_t e = threadIdx.x; e < all_heads * 64; e += kNormThreads) {
      const uint32_t word = src[e];
      const uint32_t h = e >> 6, d = (e & 63u) * 2;
      xs[h * 129 + d] = lo_bf16(word);
      xs[h * 129 + d + 1] = hi_bf16(word);
    }
  } else {
    const uint64_t slab = (uint64_t)kMaxRows * ld;
    const float* src = qkv_part + (uint64_t)row * ld;
    for (uint32_t e = threadIdx.x; e < all_heads * 128; e += kNormThreads) {
      float acc = src[e];
      for (uint32_t sp = 1; sp < splits; ++sp) acc += src[sp * slab + e];
      xs[(e >> 7) * 129 + (e & 127u)] = round_bf16(acc);
    }
  }
  __syncthreads();
  if (threadIdx.x < heads) {
    const float* xh = xs + threadIdx.x * 129;
    float sum = 0.f;
    bool bad = false;
    for (int d = 0; d < 128; ++d) {
      float a = xh[d];
      bad |= !is_finite_f32(a);
      float sq = a * a;
      sum = sum + sq;
    }
    float inv = inverse_rms(sum, 128.0f, eps);
    if (bad || !is_finite_f32(sum) || !is_finite_f32(inv)) raise_error(err, ERR_NONFINITE);
    inv_s[threadIdx.x] = inv;
  }
  __syncthreads();

  const uint32_t pos = positions[row];
  uint32_t slot_base = 0;
  bool slot_ok = pos < context && pos / 16 < stride;
  if (slot_ok) {
    uint32_t page = table[(uint64_t)row * stride + pos / 16];
    slot_ok = page < pages;
    slot_base = (page * 16u + (pos & 15u)) * kvh;
  }
  if (!slot_ok) {
    if (threadIdx.x == 0) raise_error(err, ERR_PAGE);
  }
  const uint32_t trig = (pos < context ? pos : 0) * 64;
  bool bad = false;
  for (uint32_t item = threadIdx.x; item < heads * 64; item += kNormThreads) {
    uint32_t h = item >> 6, i = item & 63u;
    const float* xh = xs + h * 129;
    const uint16_t* wn = h < qh ? q_norm : k_norm;
    float inv = inv_s[h];
    float a = bf16_to_f32(norm_weight_bf16(xh[i], inv, bf16_to_f32(wn[i])));
    float b = bf16_to_f32(norm_weight_bf16(xh[i + 64], inv, bf16_to_f32(wn[i + 64])));
    float c = cos_t[trig + i], s = sin_t[trig + i];
    float a_cos = a * c, b_sin = b * s, b_cos = b * c, a_sin = a * s;
    uint32_t ra = f32_to_bf16(a_cos - b_sin);
    uint32_t rb = f32_to_bf16(b_cos + a_sin);
    bad |= ((ra & 0x7f80u) == 0x7f80u) | ((rb & 0x7f80u) == 0x7f80u);
    if (h < qh) {
      uint16_t* qo = q_out + (uint64_t)row * qh * 128 + h * 128;
      qo[i] = (uint16_t)ra;
      qo[i + 64] = (uint16_t)rb;
    } else if (slot_ok) {
      uint16_t* ko = k_cache + ((uint64_t)slot_base + (h - qh)) * 128;
      ko[i] = (uint16_t)ra;
      ko[i + 64] = (uint16_t)rb;
    }
  }
  if (slot_ok) {
    // Raw V (neither normalized nor rotated) into the same slot.
    uint32_t* vdst = reinterpret_cast<uint32_t*>(v_cache + (uint64_t)slot_base * 128);
    for (uint32_t e = threadIdx.x; e < kvh * 64; e += kNormThreads) {
      const float* xv = xs + (heads + (e >> 6)) * 129 + (e & 63u) * 2;
      vdst[e] = f32_to_bf16(xv[0]) | (f32_to_bf16(xv[1]) << 16);
    }
  }
  if (bad) raise_error(err, ERR_NONFINITE);
}

// Residual + RMSNorm (see fh_op_residual_rmsnorm): one workgroup per row,
// 16-byte chunks c = tid, tid + 256, ... of the row.
__global__ __launch_bounds__(kNormThreads) void residual_rmsnorm_kernel(uint16_t* __restrict__ hidden,
                                                                        const float* __restrict__ part,
                                                                        uint32_t splits,
                                                                        const uint16_t* __restrict__ w,
                                                                        uint16_t* __restrict__ y, uint32_t y_tiled,
                                                                        uint32_t width, float eps, uint32_t* err) {
  __shared__ float red[kNormThreads / 64];
  const uint32_t row = blockIdx.x;
  uint16_t* hr = hidden + (uint64_t)row * width;
  const uint32_t chunks = width / 8;
  constexpr int kMaxPerThread = 4;  // width <= 8192
  const uint64_t slab = (uint64_t)kMaxRows * width;
  uint4 v[kMaxPerThread];
  float sum = 0.f;
  bool bad = false;
#pragma unroll
  for (int j = 0; j < kMaxPerThread; ++j) {
    const uint32_t c = threadIdx.x + j * kNormThreads;
    if (c < chunks) {
      v[j] = *reinterpret_cast<const uint4*>(hr + c * 8);
      if (splits) {
        // h = bf16((0 + (P_0 + P_1 + ...)) + h), v5 collective.rs:25-60 with
        // the split-K slabs added in split order.
        const float* pr = part + (uint64_t)row * width + c * 8;
        float a[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = pr[e];
        for (uint32_t sp = 1; sp < splits; ++sp)
#pragma unroll
          for (int e = 0; e < 8; ++e) a[e] += pr[sp * slab + e];
        uint32_t words[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t lo = f32_to_bf16((0.0f + a[2 * q]) + lo_bf16(words[q]));
          const uint32_t hi = f32_to_bf16((0.0f + a[2 * q + 1]) + hi_bf16(words[q]));
          words[q] = lo | (hi << 16);
        }
        v[j] = make_uint4(words[0], words[1], words[2], words[3]);
        *reinterpret_cast<uint4*>(hr + c * 8) = v[j];
      }
      const uint32_t words[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float a = lo_bf16(words[q]), b = hi_bf16(words[q]);
        bad |= !is_finite_f32(a) | !is_finite_f32(b);
        sum = sum + a * a;
        sum = sum + b * b;
      }
    }
  }
  const float total = block_sum_ordered(sum, red);
  const float inv = inverse_rms(total, (float)width, eps);
  if (!is_finite_f32(total) || !is_finite_f32(inv)) bad = true;
#pragma unroll
  for (int j = 0; j < kMaxPerThread; ++j) {
    const uint32_t c = threadIdx.x + j * kNormThreads;
    if (c < chunks) {
      const uint4 wv = *reinterpret_cast<const uint4*>(w + c * 8);
      const uint32_t xs[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
      const uint32_t ws[4] = {wv.x, wv.y, wv.z, wv.w};
      uint32_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t a = norm_weight_bf16(lo_bf16(xs[q]), inv, lo_bf16(ws[q]));
        const uint32_t b = norm_weight_bf16(hi_bf16(xs[q]), inv, hi_bf16(ws[q]));
        bad |= ((a & 0x7f80u) == 0x7f80u) | ((b & 0x7f80u) == 0x7f80u);
        o[q] = a | (b << 16);
      }
      const uint4 ov = make_uint4(o[0], o[1], o[2], o[3]);
      if (y_tiled)
        *reinterpret_cast<uint4*>(y + act_offset(row, c * 8)) = ov;
      else
        *reinterpret_cast<uint4*>(y + (uint64_t)row * width + c * 8) = ov;
    }
  }
  if (bad) raise_error(err, ERR_NONFINITE);
}

// Row-major <-> activation tile order, one 16-byte chunk per thread.
__global__ __launch_bounds__(kNormThreads) void tile_activation_kernel(const uint16_t* __restrict__ x,
                                                                       uint16_t* __restrict__ xt, uint32_t m,
                                                                       uint32_t k, uint32_t to_tiled) {
  const uint32_t chunks = m * (k / 8);
  for (uint32_t c = blockIdx.x * kNormThreads + threadIdx.x; c < chunks; c += gridDim.x * kNormThreads) {
    const uint32_t row = c / (k / 8), col = (c % (k / 8)) * 8;
    if (to_tiled)
      *reinterpret_cast<uint4*>(xt + act_offset(row, col)) =
          *reinterpret_cast<const uint4*>(x + (uint64_t)row * k + col);
    else
      *reinterpret_cast<uint4*>(const_cast<uint16_t*>(x) + (uint64_t)row * k + col) =
          *reinterpret_cast<const uint4*>(xt + act_offset(row, col));
  }
}

__global__ __launch_bounds__(kNormThreads) void swiglu_kernel(const uint16_t* __restrict__ gate,
                                                              const uint16_t* __restrict__ up,
                                                              uint16_t* __restrict__ out, uint64_t n, uint32_t* err) {
  bool bad = false;
  for (uint64_t i = (uint64_t)blockIdx.x * kNormThreads + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kNormThreads)
    out[i] = (uint16_t)swiglu_bf16(bf16_to_f32(gate[i]), bf16_to_f32(up[i]), bad);
  if (bad) raise_error(err, ERR_NONFINITE);
}

}  // namespace

hipError_t launch_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* y, uint32_t rows, uint32_t width,
                          float eps, uint32_t* err, hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kNormThreads), 0, s, x, w, y, width, eps, err);
  return hipGetLastError();
}

hipError_t launch_qknorm_rope_kv(const uint16_t* qkv, const float* qkv_part, uint32_t splits, const uint16_t* q_norm,
                                 const uint16_t* k_norm, const float* cos_t, const float* sin_t,
                                 const uint32_t* positions, const uint32_t* table, uint16_t* q_out,
                                 uint16_t* k_cache, uint16_t* v_cache, uint32_t rows, uint32_t qh, uint32_t kvh,
                                 uint32_t stride, uint32_t pages, uint32_t context, float eps, uint32_t* err,
                                 hipStream_t s) {
  size_t lds = ((size_t)(qh + 2 * kvh) * 129 + (qh + kvh)) * sizeof(float);
  hipLaunchKernelGGL(qknorm_rope_kv_kernel, dim3(rows), dim3(kNormThreads), lds, s, qkv, qkv_part, splits, q_norm,
                     k_norm, cos_t, sin_t, positions, table, q_out, k_cache, v_cache, qh, kvh, stride, pages, context,
                     eps, err);
  return hipGetLastError();
}

hipError_t launch_residual_rmsnorm(uint16_t* hidden, const float* partials, uint32_t splits, const uint16_t* w,
                                   uint16_t* y, uint32_t y_tiled, uint32_t rows, uint32_t width, float eps,
                                   uint32_t* err, hipStream_t s) {
  hipLaunchKernelGGL(residual_rmsnorm_kernel, dim3(rows), dim3(kNormThreads), 0, s, hidden, partials, splits, w, y,
                     y_tiled, width, eps, err);
  return hipGetLastError();
}

hipError_t launch_tile_activation(const uint16_t* x, uint16_t* x_tiled, uint32_t m, uint32_t k, uint32_t to_tiled,
                                  hipStream_t s) {
  const uint32_t chunks = m * (k / 8);
  const uint32_t grid = (chunks + kNormThreads - 1) / kNormThreads;
  hipLaunchKernelGGL(tile_activation_kernel, dim3(grid ? grid : 1), dim3(kNormThreads), 0, s, x, x_tiled, m, k,
                     to_tiled);
  return hipGetLastError();
}

hipError_t launch_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, uint64_t n, uint32_t* err,
                         hipStream_t s) {
  uint64_t g = (n + kNormThreads - 1) / kNormThreads;
  if (g > 65536) g = 65536;
  if (g == 0) g = 1;
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)g), dim3(kNormThreads), 0, s, gate, up, out, n, err);
  return hipGetLastError();
}

}  // namespace fh
