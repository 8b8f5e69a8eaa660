// K2 RMSNorm (wavefront reduction), K3 QK-norm + RoPE + paged KV append
// (one launch per layer), and the standalone K6 SwiGLU.
#include "common.hpp"
#include "kernels.hpp"
#include "qk_head.hpp"

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

// Per-head QK-norm, split-half RoPE and the paged KV append, fused. One
// wave per (token row, head); the heads of a row are the query heads, then
// the key heads, then the value heads of the packed QKV projection. Lane l
// owns elements l and l + 64 of its head, which is exactly one RoPE pair.
//  1. the projection output is bf16(P_0 + P_1 + ... + P_{S-1}) over the
//     split-K slabs, added in split order and rounded once (the reference's
//     one RNE per projection output), or the bf16 row itself (S = 0);
//  2. q and k heads: the sum of squares runs serially in ascending element
//     order (readlane chain), which is exactly qwen3_rmsnorm_v1 at width 128
//     (rmsnorm.rs:421-438, as called for QK-norm at
//     tp_execution/batched.rs:1956-1982);
//  3. bf16(bf16(x*inv)*w) for both halves, then the RoPE pair with separately
//     rounded products (rope_kv.rs:102-240, v5 rope_kv.rs:60-80):
//     a' = a*c - b*s, b' = b*c + a*s, each narrowed once;
//  4. rotated k and raw v go to cache[(page*16 + pos%16)][kv_head][128], the
//     slot of qwen3_paged_kv_write_v1 (rope_kv.rs:261-388).
// S < 0 takes the split count from the argument (any count); S > 0 fixes it
// at compile time so every slab load of a lane is in flight at once.
constexpr int kHeadsPerGroup = 4;

template <int S>
__global__ __launch_bounds__(kHeadsPerGroup * 64) void qknorm_rope_kv_kernel(
    const uint16_t* __restrict__ qkv, const float* __restrict__ qkv_part, uint32_t splits,
    const uint16_t* __restrict__ q_norm, const uint16_t* __restrict__ k_norm, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, const uint32_t* __restrict__ positions, const uint32_t* __restrict__ table,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache, uint32_t qh,
    uint32_t kvh, uint32_t stride, uint32_t pages, uint32_t context, float eps, uint32_t slab_rows, uint32_t* err) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t head = blockIdx.x * kHeadsPerGroup + (threadIdx.x >> 6);
  const uint32_t row = blockIdx.y;
  const uint32_t heads = qh + kvh;  // normalized and rotated heads
  if (head >= heads + kvh) return;
  const uint32_t ld = (heads + kvh) * 128;
  const uint64_t base = (uint64_t)row * ld + head * 128 + lane;

  float a, b;
  if constexpr (S == 0) {
    a = bf16_to_f32(qkv[base]);
    b = bf16_to_f32(qkv[base + 64]);
  } else {
    const uint64_t slab = (uint64_t)slab_rows * ld;
    if constexpr (S > 0) {
      float pa[S], pb[S];
#pragma unroll
      for (int sp = 0; sp < S; ++sp) {
        pa[sp] = qkv_part[sp * slab + base];
        pb[sp] = qkv_part[sp * slab + base + 64];
      }
      a = pa[0];
      b = pb[0];
#pragma unroll
      for (int sp = 1; sp < S; ++sp) {
        a += pa[sp];
        b += pb[sp];
      }
    } else {
      a = qkv_part[base];
      b = qkv_part[base + 64];
      for (uint32_t sp = 1; sp < splits; ++sp) {
        a += qkv_part[sp * slab + base];
        b += qkv_part[sp * slab + base + 64];
      }
    }
    a = round_bf16(a);
    b = round_bf16(b);
  }

  const uint32_t pos = positions[row];
  uint32_t slot = 0;
  bool slot_ok = pos < context && pos / 16 < stride;
  if (slot_ok) {
    const uint32_t page = table[(uint64_t)row * stride + pos / 16];
    slot_ok = page < pages;
    slot = (page * 16u + (pos & 15u)) * kvh;
  }
  if (!slot_ok && head == 0 && lane == 0) raise_error(err, ERR_PAGE);

  if (head >= heads) {
    // Raw V (neither normalized nor rotated) into the slot.
    if (slot_ok) {
      uint16_t* vo = v_cache + ((uint64_t)slot + (head - heads)) * 128;
      vo[lane] = (uint16_t)f32_to_bf16(a);
      vo[lane + 64] = (uint16_t)f32_to_bf16(b);
    }
    return;
  }

  const uint16_t* wn = head < qh ? q_norm : k_norm;
  const uint32_t trig = (pos < context ? pos : 0) * 64 + lane;
  uint32_t ra, rb;
  const bool bad = qknorm_rope_wave_head(a, b, bf16_to_f32(wn[lane]), bf16_to_f32(wn[lane + 64]), cos_t[trig],
                                         sin_t[trig], eps, ra, rb);
  uint16_t* dst = nullptr;
  if (head < qh)
    dst = q_out + ((uint64_t)row * qh + head) * 128;
  else if (slot_ok)
    dst = k_cache + ((uint64_t)slot + (head - qh)) * 128;
  if (dst) {
    dst[lane] = (uint16_t)ra;
    dst[lane + 64] = (uint16_t)rb;
  }
  if (bad) raise_error(err, ERR_NONFINITE);
}

// Residual + RMSNorm (see fh_op_residual_rmsnorm): one workgroup per row,
// 16-byte chunks c = tid, tid + 256, ... of the row (CH of them per thread,
// width <= CH * 2048). S as in the QK-norm kernel: 0 = no partials, > 0 =
// compile-time split count, < 0 = any count.
template <int S, int CH>
__global__ __launch_bounds__(kNormThreads) void residual_rmsnorm_kernel(uint16_t* __restrict__ hidden,
                                                                        const float* __restrict__ part,
                                                                        uint32_t splits,
                                                                        const uint16_t* __restrict__ w,
                                                                        uint16_t* __restrict__ y, uint32_t y_mtiles,
                                                                        uint32_t width, float eps, uint32_t slab_rows,
                                                                        uint32_t* err) {
  __shared__ float red[kNormThreads / 64];
  const uint32_t row = blockIdx.x;
  uint16_t* hr = hidden + (uint64_t)row * width;
  const uint32_t chunks = width / 8;
  const uint64_t slab = (uint64_t)slab_rows * width;
  const uint64_t slab4 = slab / 4;
  // With a compile-time split count every chunk's row and slab loads are
  // issued before the first fold (one memory round trip for the whole row)
  // while the slab registers stay within 128 VGPRs; the arithmetic and its
  // order are the same either way.
  constexpr bool kLoadsFirst = S > 0 && CH * S <= 16;
  uint4 v[CH], wv[CH];
  float4 pre[kLoadsFirst ? CH : 1][kLoadsFirst ? S : 1][2];
  float sum = 0.f;
  bool bad = false;
  // The norm weight is loaded with the row, not after the reduction: one
  // memory round trip less on this latency-bound kernel.
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const uint32_t c = threadIdx.x + j * kNormThreads;
    if (c < chunks) wv[j] = *reinterpret_cast<const uint4*>(w + c * 8);
  }
  if constexpr (kLoadsFirst) {
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const uint32_t c = threadIdx.x + j * kNormThreads;
      if (c < chunks) {
        v[j] = *reinterpret_cast<const uint4*>(hr + c * 8);
        const float4* pr = reinterpret_cast<const float4*>(part + (uint64_t)row * width + c * 8);
#pragma unroll
        for (int sp = 0; sp < S; ++sp) {
          pre[j][sp][0] = pr[sp * slab4];
          pre[j][sp][1] = pr[sp * slab4 + 1];
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const uint32_t c = threadIdx.x + j * kNormThreads;
    if (c < chunks) {
      if constexpr (!kLoadsFirst) v[j] = *reinterpret_cast<const uint4*>(hr + c * 8);
      if constexpr (S != 0) {
        // h = bf16((0 + (P_0 + P_1 + ...)) + h), v5 collective.rs:25-60 with
        // the split-K slabs added in split order.
        const float4* pr = reinterpret_cast<const float4*>(part + (uint64_t)row * width + c * 8);
        float a[8];
        if constexpr (S > 0) {
          float4 p[S][2];
#pragma unroll
          for (int sp = 0; sp < S; ++sp) {
            if constexpr (kLoadsFirst) {
              p[sp][0] = pre[j][sp][0];
              p[sp][1] = pre[j][sp][1];
            } else {
              p[sp][0] = pr[sp * slab4];
              p[sp][1] = pr[sp * slab4 + 1];
            }
          }
          a[0] = p[0][0].x; a[1] = p[0][0].y; a[2] = p[0][0].z; a[3] = p[0][0].w;
          a[4] = p[0][1].x; a[5] = p[0][1].y; a[6] = p[0][1].z; a[7] = p[0][1].w;
#pragma unroll
          for (int sp = 1; sp < S; ++sp) {
            a[0] += p[sp][0].x; a[1] += p[sp][0].y; a[2] += p[sp][0].z; a[3] += p[sp][0].w;
            a[4] += p[sp][1].x; a[5] += p[sp][1].y; a[6] += p[sp][1].z; a[7] += p[sp][1].w;
          }
        } else {
          const float* pf = reinterpret_cast<const float*>(pr);
#pragma unroll
          for (int e = 0; e < 8; ++e) a[e] = pf[e];
          for (uint32_t sp = 1; sp < splits; ++sp)
#pragma unroll
            for (int e = 0; e < 8; ++e) a[e] += pf[sp * slab + e];
        }
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
  for (int j = 0; j < CH; ++j) {
    const uint32_t c = threadIdx.x + j * kNormThreads;
    if (c < chunks) {
      const uint32_t xs[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
      const uint32_t ws[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
      uint32_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t a = norm_weight_bf16(lo_bf16(xs[q]), inv, lo_bf16(ws[q]));
        const uint32_t b = norm_weight_bf16(hi_bf16(xs[q]), inv, hi_bf16(ws[q]));
        bad |= ((a & 0x7f80u) == 0x7f80u) | ((b & 0x7f80u) == 0x7f80u);
        o[q] = a | (b << 16);
      }
      const uint4 ov = make_uint4(o[0], o[1], o[2], o[3]);
      if (y_mtiles)
        *reinterpret_cast<uint4*>(y + act_offset_m(row, c * 8, y_mtiles)) = ov;
      else
        *reinterpret_cast<uint4*>(y + (uint64_t)row * width + c * 8) = ov;
    }
  }
  if (bad) raise_error(err, ERR_NONFINITE);
}

// The same computation for bf16 QKV rows (S = 0, the prefill path), one
// lane per (row, head) (qk_head.hpp): the lane holds the head's 128 values
// and runs the serial sum of squares (ascending element order, each square
// rounded before the add, exactly as above) itself, so no cross-lane chain
// limits a chunk of thousands of rows. Value heads are copied raw into the
// slot.
__global__ __launch_bounds__(256, 2) void qknorm_rope_kv_rows_kernel(const uint16_t* __restrict__ qkv, QkvRopeArgs a,
                                                                     uint32_t rows) {
  const uint32_t all = a.qh + 2 * a.kvh;
  const uint64_t gid = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (uint64_t)rows * all) return;
  const uint32_t row = (uint32_t)(gid / all), head = (uint32_t)(gid % all);
  qknorm_rope_kv_head(reinterpret_cast<const qk_u32x4*>(qkv + (uint64_t)row * all * 128 + (uint64_t)head * 128), row,
                      head, a, qkv_row_slot(row, a));
}

// RMSNorm of many rows into activation tile order (the prefill path, no
// split-K partials): one 512-thread workgroup per 16-row tile. Thread t
// handles the tile-order chunks q = 512 j + t of its row tile (k-block
// q / 64, in-tile lane q % 64, i.e. row q % 16, columns 32 (q / 64) +
// 8 ((q % 64) / 16)), so every wave writes whole 1 KiB tiles and reads 64
// contiguous bytes of each of 16 rows (a tile written piecewise by
// different waves would cost partial-line writes). All of a thread's
// chunks belong to row t % 16: the row's sum of squares is the thread
// partials (chunks in ascending j) added over t = r, r + 16, ... in order.
// The norm weight is staged in LDS with the row loads, so the output pass
// waits for no second memory round trip. width % 32 == 0, width <= 4096.
constexpr uint32_t kTileRows = 16;
constexpr int kTileThreads = 512;
constexpr int kRowsMaxChunks = 4096 / 8 * kTileRows / kTileThreads;  // 16

__global__ __launch_bounds__(kTileThreads) void rmsnorm_tile_rows_kernel(const uint16_t* __restrict__ x,
                                                                         const uint16_t* __restrict__ w,
                                                                         uint16_t* __restrict__ y, uint32_t rows,
                                                                         uint32_t y_mtiles, uint32_t width, float eps,
                                                                         uint32_t* err) {
  __shared__ float part[kTileThreads];
  __shared__ float inv_s[kTileRows];
  __shared__ uint32_t bad_s;
  __shared__ uint4 w_s[4096 / 8];
  const uint32_t t = threadIdx.x, mt = blockIdx.x, row0 = mt * kTileRows;
  const uint32_t lane = t & 63u, r = lane & 15u, g = lane >> 4;
  const uint32_t kbs = width / 32;  // k-blocks per row
  const bool live = row0 + r < rows;
  if (t == 0) bad_s = 0;
  for (uint32_t c = t; c < width / 8; c += kTileThreads) w_s[c] = *reinterpret_cast<const uint4*>(w + c * 8);
  uint4 v[kRowsMaxChunks];
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < kRowsMaxChunks; ++j) {
    const uint32_t kb = j * (kTileThreads / 64) + (t >> 6);
    if (kb < kbs && live) {
      v[j] = *reinterpret_cast<const uint4*>(x + (uint64_t)(row0 + r) * width + kb * 32 + g * 8);
      const uint32_t words[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float a = lo_bf16(words[k]), b = hi_bf16(words[k]);
        sum = sum + a * a;
        sum = sum + b * b;
      }
    } else {
      v[j] = make_uint4(0u, 0u, 0u, 0u);
    }
  }
  part[t] = sum;
  __syncthreads();
  if (t < kTileRows) {
    float s2 = part[t];
    for (uint32_t i = 1; i < kTileThreads / kTileRows; ++i) s2 = s2 + part[t + kTileRows * i];
    const float inv = inverse_rms(s2, (float)width, eps);
    inv_s[t] = inv;
    if (row0 + t < rows && (!is_finite_f32(s2) || !is_finite_f32(inv))) bad_s = 1;
  }
  __syncthreads();
  bool bad = false;
  const float inv = inv_s[r];
#pragma unroll
  for (int j = 0; j < kRowsMaxChunks; ++j) {
    const uint32_t kb = j * (kTileThreads / 64) + (t >> 6);
    if (kb < kbs) {
      uint32_t o[4] = {0u, 0u, 0u, 0u};
      if (live) {
        const uint4 wv = w_s[kb * 4 + g];
        const uint32_t xs[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
        const uint32_t ws[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t a = norm_weight_bf16(lo_bf16(xs[k]), inv, lo_bf16(ws[k]));
          const uint32_t b = norm_weight_bf16(hi_bf16(xs[k]), inv, hi_bf16(ws[k]));
          bad |= ((a & 0x7f80u) == 0x7f80u) | ((b & 0x7f80u) == 0x7f80u);
          o[k] = a | (b << 16);
        }
      }
      // Rows past the batch in the last tile are written as zeros (the tiled
      // buffer's padding rows, which the projections read and never use).
      *reinterpret_cast<uint4*>(y + (((uint64_t)kb * y_mtiles + mt) * 64 + lane) * 8) =
          make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
  if (bad || (t == 0 && bad_s)) raise_error(err, ERR_NONFINITE);
}

// Row-major <-> activation tile order, one 16-byte chunk per thread.
__global__ __launch_bounds__(kNormThreads) void tile_activation_kernel(const uint16_t* __restrict__ x,
                                                                       uint16_t* __restrict__ xt, uint32_t m,
                                                                       uint32_t k, uint32_t to_tiled,
                                                                       uint32_t mtiles) {
  const uint32_t chunks = m * (k / 8);
  for (uint32_t c = blockIdx.x * kNormThreads + threadIdx.x; c < chunks; c += gridDim.x * kNormThreads) {
    const uint32_t row = c / (k / 8), col = (c % (k / 8)) * 8;
    if (to_tiled)
      *reinterpret_cast<uint4*>(xt + act_offset_m(row, col, mtiles)) =
          *reinterpret_cast<const uint4*>(x + (uint64_t)row * k + col);
    else
      *reinterpret_cast<uint4*>(const_cast<uint16_t*>(x) + (uint64_t)row * k + col) =
          *reinterpret_cast<const uint4*>(xt + act_offset_m(row, col, mtiles));
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

// Row counts up to which the norms run one wave or workgroup per row (and
// head) rather than the many-row kernels.
constexpr uint32_t kWaveNormRows = 256;

hipError_t launch_qknorm_rope_kv(const uint16_t* qkv, const float* qkv_part, uint32_t splits, const uint16_t* q_norm,
                                 const uint16_t* k_norm, const float* cos_t, const float* sin_t,
                                 const uint32_t* positions, const uint32_t* table, uint16_t* q_out,
                                 uint16_t* k_cache, uint16_t* v_cache, uint32_t rows, uint32_t qh, uint32_t kvh,
                                 uint32_t stride, uint32_t pages, uint32_t context, float eps, uint32_t* err,
                                 hipStream_t s) {
  // bf16 rows: up to 256 rows one wave per (row, head) as in decode (the
  // 8B shape at 160 rows: 6400 waves); beyond that one lane per (row, head).
  if (!qkv_part && rows > kWaveNormRows) {
    const uint64_t lanes = (uint64_t)rows * (qh + 2 * kvh);
    const QkvRopeArgs a{q_norm, k_norm, cos_t, sin_t, positions, table, q_out, k_cache, v_cache,
                        qh,     kvh,    stride, pages, context, eps,   err};
    hipLaunchKernelGGL(qknorm_rope_kv_rows_kernel, dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0, s, qkv, a, rows);
    return hipGetLastError();
  }
  const dim3 grid((qh + 2 * kvh + kHeadsPerGroup - 1) / kHeadsPerGroup, rows);
  const dim3 block(kHeadsPerGroup * 64);
#define FH_QKNORM(S_)                                                                                              \
  hipLaunchKernelGGL(qknorm_rope_kv_kernel<S_>, grid, block, 0, s, qkv, qkv_part, splits, q_norm, k_norm, cos_t,  \
                     sin_t, positions, table, q_out, k_cache, v_cache, qh, kvh, stride, pages, context, eps,           \
                     partial_slab_rows(rows), err)
  switch (qkv_part ? splits : 0) {
    case 0: FH_QKNORM(0); break;
    case 1: FH_QKNORM(1); break;
    case 2: FH_QKNORM(2); break;
    case 3: FH_QKNORM(3); break;
    case 4: FH_QKNORM(4); break;
    case 5: FH_QKNORM(5); break;
    case 6: FH_QKNORM(6); break;
    case 8: FH_QKNORM(8); break;
    default: FH_QKNORM(-1); break;
  }
#undef FH_QKNORM
  return hipGetLastError();
}

hipError_t launch_residual_rmsnorm(uint16_t* hidden, const float* partials, uint32_t splits, const uint16_t* w,
                                   uint16_t* y, uint32_t y_tiled, uint32_t rows, uint32_t width, float eps,
                                   uint32_t* err, hipStream_t s) {
  // One workgroup per row up to 256 rows (160 rows: 160 workgroups, where
  // the 16-row-tile kernel would run 10), one per 16-row tile beyond.
  if (!partials && y_tiled && rows > kWaveNormRows && width % 32 == 0 && width <= 4096) {
    hipLaunchKernelGGL(rmsnorm_tile_rows_kernel, dim3((rows + kTileRows - 1) / kTileRows), dim3(kTileThreads), 0, s,
                       hidden, w, y, rows, act_mtiles(rows), width, eps, err);
    return hipGetLastError();
  }
  const uint32_t per_thread = (width / 8 + kNormThreads - 1) / kNormThreads;  // 16-byte chunks
#define FH_RESNORM_CH(S_, CH_)                                                                                     \
  hipLaunchKernelGGL((residual_rmsnorm_kernel<S_, CH_>), dim3(rows), dim3(kNormThreads), 0, s, hidden, partials,  \
                     splits, w, y, y_tiled ? act_mtiles(rows) : 0u, width, eps, partial_slab_rows(rows), err)
#define FH_RESNORM(S_)                   \
  if (per_thread <= 1)                   \
    FH_RESNORM_CH(S_, 1);                \
  else if (per_thread <= 2)              \
    FH_RESNORM_CH(S_, 2);                \
  else                                   \
    FH_RESNORM_CH(S_, 4)
  switch (partials ? splits : 0) {
    case 0: FH_RESNORM(0); break;
    case 1: FH_RESNORM(1); break;
    case 2: FH_RESNORM(2); break;
    case 3: FH_RESNORM(3); break;
    case 4: FH_RESNORM(4); break;
    case 6: FH_RESNORM(6); break;
    case 8: FH_RESNORM(8); break;
    default: FH_RESNORM(-1); break;
  }
#undef FH_RESNORM
#undef FH_RESNORM_CH
  return hipGetLastError();
}

hipError_t launch_tile_activation(const uint16_t* x, uint16_t* x_tiled, uint32_t m, uint32_t k, uint32_t to_tiled,
                                  hipStream_t s) {
  const uint32_t chunks = m * (k / 8);
  const uint32_t grid = (chunks + kNormThreads - 1) / kNormThreads;
  hipLaunchKernelGGL(tile_activation_kernel, dim3(grid ? grid : 1), dim3(kNormThreads), 0, s, x, x_tiled, m, k,
                     to_tiled, act_mtiles(m));
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
