// K1 projections for decode (m <= 32 token rows): weight-streaming GEMM on
// gfx950 MFMA (v_mfma_f32_16x16x32_bf16) with FP32 accumulation; for 33..256
// rows the same weight stream against an activation panel shared through LDS
// (gemm_panel_kernel below).
//
// Data layout. The weight W[n][k] is stored in MFMA tile order (common.hpp
// tiled_offset) and the activation x[m][k] in activation tile order
// (common.hpp act_offset): every operand load of a wave is one contiguous,
// fully coalesced 1 KiB that lands directly in the MFMA's A or B registers —
// no LDS staging, no transposes, no partially used cache lines.
//
// Work split. A wave owns NT consecutive 16-row n-tiles (NT = 4: 64 weight
// rows share each activation load, so activation traffic is half the weight
// traffic at m = 32). Grid = (n / (16 NT), splits): blockIdx.y selects a
// contiguous range of k-blocks, and the WAVES waves of a workgroup split that
// range again. Wave partials are added in wave order through LDS
// (deterministic). Epilogues:
//   FH_EPI_PARTIAL  FP32 partial sums, one [partial_slab_rows(m)][ldo] slab per split; the
//                    consumer adds the slabs in split order and rounds once
//                    (residual + RMSNorm, QK-norm) — no atomics, no extra launch
//   FH_EPI_BF16     out = bf16(acc)                       (gemm.rs:161 beta = 0)
//   FH_EPI_RESIDUAL out = bf16((0 + acc) + residual)      (v5 collective.rs:25-60)
//   FH_EPI_SWIGLU   act = swiglu(bf16(gate), bf16(up)), written in activation
//                    tile order for the down projection; tiles 2j / 2j+1 are
//                    gate / up of the same 16 columns (K6 fused, swiglu.rs:62-101)
//   FH_EPI_F32      out = acc                              (FP32 LM head, v8 projection.rs:66)
// Rounding points are the reference's (one bf16 RNE per projection output;
// gate and up narrowed before SwiGLU); the FP32 summation order is
// reassociated (32-wide MFMA k-blocks, wave ranges, splits), as the
// reference's own wave and MFMA profiles reassociate (v5 projection.rs:15, :241).
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"
#include "../../include/ferric_hip.h"

namespace fh {

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8 as_b8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

constexpr int kRowNormThreads = 256;  // the residual + RMSNorm kernel's thread count and mapping

// Batches of more than 32 rows run as 32-row chunks (gridDim.z of them, one
// split): every chunk streams the same weight tiles.
//
// NS >= 0 (one row): the row's residual + RMSNorm runs in the prologue of
// every workgroup (RowNormArgs; NS split-K slabs folded, NJ 16-byte chunks
// per thread), with the norm kernel's thread mapping and reduction order
// (threads 0..255: chunks t, t + 256, ...; squares summed per thread in chunk
// order, then the four wave totals in wave order), so x is bit-identical to
// that kernel's. The prologue's loads go out first and the first weight
// chunk's right after them, so the weights stream while the row is folded
// and reduced; x is staged in LDS and each k-block's B operand is read from
// there (lanes 0, 16, 32, 48 hold row 0; the other 15 rows of the tile are
// zero: they only produce the discarded output rows).
template <int NT, int MT, int EPI, int WAVES, int UNROLL, int NS = -1, int NJ = 1>
__global__ __launch_bounds__(WAVES * 64) void gemm_kernel(const uint16_t* __restrict__ xt,
                                                         const uint16_t* __restrict__ w, uint32_t m_total,
                                                         uint32_t kb_count, uint32_t kb_split, uint32_t x_mtiles,
                                                         const uint16_t* residual, void* out, uint32_t ldo,
                                                         uint32_t* err, RowNormArgs na) {
  constexpr bool kNorm = NS >= 0;
  static_assert(!kNorm || MT == 1, "the fused norm serves one row");
  static_assert(!kNorm || WAVES * 64 >= kRowNormThreads, "the norm's 256-thread mapping");
  __shared__ float red[WAVES][NT * MT * 256];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // A launch over several 32-row chunks (always one split) reads each weight
  // slice once per chunk. Workgroups go to the 8 XCDs round-robin by
  // dispatch order, so the order is arranged for the chunks of one slice to
  // be dispatched back to back on one XCD: they run together there and the
  // later ones find the weight tiles in that XCD's L2. Slices past the last
  // multiple of 8 keep their chunks consecutive in dispatch order.
  uint32_t slice = blockIdx.x, chunk = blockIdx.z;
  if (gridDim.z > 1) {
    const uint32_t S = gridDim.x, C = gridDim.z, S8 = S & ~7u;
    const uint32_t b = blockIdx.x + S * blockIdx.z;
    if (b < S8 * C) {
      const uint32_t r = b >> 3;
      chunk = r % C;
      slice = (r / C) * 8 + (b & 7u);
    } else {
      const uint32_t t = b - S8 * C;
      slice = S8 + t / C;
      chunk = t % C;
    }
  }
  const uint32_t tile0 = slice * NT;
  const uint32_t split = blockIdx.y;
  const uint32_t s_lo = split * kb_split;
  const uint32_t s_hi = min(s_lo + kb_split, kb_count);
  const uint32_t s_n = s_hi > s_lo ? s_hi - s_lo : 0;
  const uint32_t kb_lo = s_lo + (s_n * wave) / WAVES;
  const uint32_t kb_hi = s_lo + (s_n * (wave + 1)) / WAVES;

  const u32x4* wp[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
    wp[nt] = reinterpret_cast<const u32x4*>(w) + ((uint64_t)(tile0 + nt) * kb_count + kb_lo) * 64 + lane;
  const uint32_t row0 = chunk * 16 * MT;
  const uint32_t m = min(m_total - row0, 16u * MT);
  const uint64_t xkb = (uint64_t)x_mtiles * 64;  // 16-byte units per k-block of the activation
  const u32x4* xp = reinterpret_cast<const u32x4*>(xt) + (uint64_t)kb_lo * xkb + chunk * MT * 64 + lane;

  f32x4 acc[NT][MT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const uint32_t steps = kb_hi - kb_lo;
  const uint32_t chunks = steps / UNROLL;
  // Each wave walks the whole-chunk part of its k-range starting at a
  // rotated k-block (and wrapping). With every wave starting at the same
  // aligned offset of its 1 KiB-tile streams, the concurrent loads of the
  // grid fall on the same HBM channels and a 200 MB stream runs at ~5.2 TB/s
  // instead of ~6.3; staggered starts spread them. The rotation depends on
  // the launch coordinates only, so the summation order of an output does
  // not depend on the batch's row count.
  const uint32_t whole = chunks * UNROLL;
  const uint32_t rot = whole ? ((slice * WAVES + wave) * 7u + blockIdx.y * 5u) % whole : 0u;
  // Software pipeline over chunks of UNROLL k-blocks with two register sets:
  // the next chunk's loads are issued before the current chunk's MFMAs, and
  // scheduling barriers keep the compiler from sinking them back next to
  // their uses (which would leave one or two loads in flight per wave).
  u32x4 wa[UNROLL][NT], xa[UNROLL][MT], wb[UNROLL][NT], xb[UNROLL][MT];
  // Fused norm: the normalized row in LDS, 8 bf16 per entry (k / 8 entries).
  __shared__ __attribute__((aligned(16))) u32x4 xs[kNorm ? NJ * kRowNormThreads : 1];
  __shared__ float nred[kRowNormThreads / 64];
  // B operand of k-block kb_lo + sk from the staged row.
  auto norm_x = [&](uint32_t sk) {
    const u32x4 v = xs[(kb_lo + sk) * 4 + (lane >> 4)];
    return (lane & 15) == 0 ? v : u32x4{0u, 0u, 0u, 0u};
  };
  auto load = [&](u32x4(&wv)[UNROLL][NT], u32x4(&xv)[UNROLL][MT], uint32_t s0) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      uint32_t sk = s0 + u + rot;
      if (sk >= whole) sk -= whole;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) wv[u][nt] = __builtin_nontemporal_load(wp[nt] + (uint64_t)sk * 64);
      if constexpr (kNorm) {
        xv[u][0] = norm_x(sk);
      } else {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) xv[u][mt] = xp[(uint64_t)sk * xkb + mt * 64];
      }
    }
  };
  auto compute = [&](u32x4(&wv)[UNROLL][NT], u32x4(&xv)[UNROLL][MT]) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(wv[u][nt]), as_b8(xv[u][mt]), acc[nt][mt], 0, 0, 0);
  };
  if constexpr (kNorm) {
    // Prologue loads (norm weight, residual row, slabs), then the first
    // weight chunk, then the fold and the reduction.
    const int t = threadIdx.x;
    const uint32_t width = kb_count * 32, nchunks = width / 8;
    const uint64_t slab = (uint64_t)na.slab_rows * width;
    uint4 hv[NJ], wv8[NJ];
    float4 pv[NJ][NS > 0 ? NS : 1][2];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t c = t + j * kRowNormThreads;
      if (t < kRowNormThreads && c < nchunks) wv8[j] = *reinterpret_cast<const uint4*>(na.w + c * 8);
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t c = t + j * kRowNormThreads;
      if (t < kRowNormThreads && c < nchunks) {
        hv[j] = *reinterpret_cast<const uint4*>(na.hidden_in + c * 8);
        if constexpr (NS > 0) {
          const float4* pr = reinterpret_cast<const float4*>(na.part + c * 8);
#pragma unroll
          for (int sp = 0; sp < NS; ++sp) {
            pv[j][sp][0] = pr[sp * (slab / 4)];
            pv[j][sp][1] = pr[sp * (slab / 4) + 1];
          }
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (chunks > 0) {
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        uint32_t sk = u + rot;
        if (sk >= whole) sk -= whole;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) wa[u][nt] = __builtin_nontemporal_load(wp[nt] + (uint64_t)sk * 64);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    float sum = 0.f;
    bool bad = false;
    const bool writer = NS > 0 && blockIdx.x == 0 && blockIdx.y == 0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t c = t + j * kRowNormThreads;
      if (t < kRowNormThreads && c < nchunks) {
        if constexpr (NS > 0) {
          // h = bf16((0 + (P_0 + P_1 + ...)) + h), the slabs in split order.
          float a[8] = {pv[j][0][0].x, pv[j][0][0].y, pv[j][0][0].z, pv[j][0][0].w,
                        pv[j][0][1].x, pv[j][0][1].y, pv[j][0][1].z, pv[j][0][1].w};
#pragma unroll
          for (int sp = 1; sp < NS; ++sp) {
            a[0] += pv[j][sp][0].x; a[1] += pv[j][sp][0].y; a[2] += pv[j][sp][0].z; a[3] += pv[j][sp][0].w;
            a[4] += pv[j][sp][1].x; a[5] += pv[j][sp][1].y; a[6] += pv[j][sp][1].z; a[7] += pv[j][sp][1].w;
          }
          uint32_t words[4] = {hv[j].x, hv[j].y, hv[j].z, hv[j].w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t lo = f32_to_bf16((0.0f + a[2 * q]) + lo_bf16(words[q]));
            const uint32_t hi = f32_to_bf16((0.0f + a[2 * q + 1]) + hi_bf16(words[q]));
            words[q] = lo | (hi << 16);
          }
          hv[j] = make_uint4(words[0], words[1], words[2], words[3]);
          if (writer) *reinterpret_cast<uint4*>(na.hidden_out + c * 8) = hv[j];
        }
        const uint32_t words[4] = {hv[j].x, hv[j].y, hv[j].z, hv[j].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float x0 = lo_bf16(words[q]), x1 = hi_bf16(words[q]);
          bad |= !is_finite_f32(x0) | !is_finite_f32(x1);
          sum = sum + x0 * x0;
          sum = sum + x1 * x1;
        }
      }
    }
    // The four wave totals of threads 0..255, in wave order.
    sum = wave_sum(sum);
    if (lane == 0 && t < kRowNormThreads) nred[t >> 6] = sum;
    __syncthreads();
    float total = nred[0];
#pragma unroll
    for (int q = 1; q < kRowNormThreads / 64; ++q) total += nred[q];
    const float inv = inverse_rms(total, (float)width, na.eps);
    if (!is_finite_f32(total) || !is_finite_f32(inv)) bad = true;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t c = t + j * kRowNormThreads;
      if (t < kRowNormThreads && c < nchunks) {
        const uint32_t xw[4] = {hv[j].x, hv[j].y, hv[j].z, hv[j].w};
        const uint32_t ww[4] = {wv8[j].x, wv8[j].y, wv8[j].z, wv8[j].w};
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t lo = norm_weight_bf16(lo_bf16(xw[q]), inv, lo_bf16(ww[q]));
          const uint32_t hi = norm_weight_bf16(hi_bf16(xw[q]), inv, hi_bf16(ww[q]));
          bad |= ((lo & 0x7f80u) == 0x7f80u) | ((hi & 0x7f80u) == 0x7f80u);
          o[q] = lo | (hi << 16);
        }
        xs[c] = u32x4{o[0], o[1], o[2], o[3]};
      }
    }
    // One workgroup reports what every workgroup sees the same way.
    if (bad && blockIdx.x == 0 && blockIdx.y == 0) raise_error(err, ERR_NONFINITE);
    __syncthreads();
    if (chunks > 0) {
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        uint32_t sk = u + rot;
        if (sk >= whole) sk -= whole;
        xa[u][0] = norm_x(sk);
      }
    }
  } else {
    if (chunks > 0) load(wa, xa, 0);
  }
  for (uint32_t c = 0; c < chunks; c += 2) {
    if (c + 1 < chunks) load(wb, xb, (c + 1) * UNROLL);
    __builtin_amdgcn_sched_barrier(0);
    compute(wa, xa);
    __builtin_amdgcn_sched_barrier(0);
    if (c + 1 < chunks) {
      if (c + 2 < chunks) load(wa, xa, (c + 2) * UNROLL);
      __builtin_amdgcn_sched_barrier(0);
      compute(wb, xb);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  uint32_t s = chunks * UNROLL;
  for (; s < steps; ++s) {
    u32x4 wv[NT], xv[MT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) wv[nt] = __builtin_nontemporal_load(wp[nt] + (uint64_t)s * 64);
    if constexpr (kNorm) {
      xv[0] = norm_x(s);
    } else {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) xv[mt] = xp[(uint64_t)s * xkb + mt * 64];
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(wv[nt]), as_b8(xv[mt]), acc[nt][mt], 0, 0, 0);
  }

  // D layout of the 16x16 MFMA: lane l, element e holds row i = 4*(l/16) + e
  // (weight row n) and column j = l % 16 (activation row m). Stored
  // transposed as [j][i] so the epilogue walks n fastest.
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        red[wave][(nt * MT + mt) * 256 + (lane & 15) * 16 + 4 * (lane >> 4) + e] = acc[nt][mt][e];
  __syncthreads();

  if constexpr (EPI == FH_EPI_SWIGLU) {
    static_assert(NT % 2 == 0, "SwiGLU epilogue pairs a gate tile with an up tile");
    bool bad = false;
    for (int idx = threadIdx.x; idx < (NT / 2) * MT * 256; idx += WAVES * 64) {
      const int pair = idx / (MT * 256), rem = idx % (MT * 256);
      const int mt = rem >> 8, j = (rem >> 4) & 15, i = rem & 15;
      const uint32_t row = mt * 16 + j;
      const int gi = ((2 * pair) * MT + mt) * 256 + j * 16 + i;
      const int ui = ((2 * pair + 1) * MT + mt) * 256 + j * 16 + i;
      float g = red[0][gi], u = red[0][ui];
#pragma unroll
      for (int wv = 1; wv < WAVES; ++wv) {
        g += red[wv][gi];
        u += red[wv][ui];
      }
      if (row < m) {
        const uint32_t col = (tile0 / 2 + pair) * 16 + i;
        const uint32_t y = swiglu_bf16(round_bf16(g), round_bf16(u), bad);
        reinterpret_cast<uint16_t*>(out)[act_offset_m(row0 + row, col, act_mtiles(m_total))] = (uint16_t)y;
      }
    }
    if (bad) raise_error(err, ERR_NONFINITE);
  } else {
    for (int idx = threadIdx.x; idx < NT * MT * 256; idx += WAVES * 64) {
      const int tm = idx >> 8, j = (idx >> 4) & 15, i = idx & 15;
      const int nt = tm / MT, mt = tm % MT;
      const uint32_t row = mt * 16 + j;
      float v = red[0][idx];
#pragma unroll
      for (int wv = 1; wv < WAVES; ++wv) v += red[wv][idx];
      if (row >= m) continue;
      const uint64_t n = (uint64_t)(tile0 + nt) * 16 + i;
      const uint64_t o = (uint64_t)(row0 + row) * ldo + n;
      if constexpr (EPI == FH_EPI_PARTIAL) {
        reinterpret_cast<float*>(out)[(uint64_t)split * kMaxRows * ldo + o] = v;
      } else if constexpr (EPI == FH_EPI_BF16) {
        reinterpret_cast<uint16_t*>(out)[o] = (uint16_t)f32_to_bf16(v);
      } else if constexpr (EPI == FH_EPI_RESIDUAL) {
        const float r = bf16_to_f32(residual[o]);
        reinterpret_cast<uint16_t*>(out)[o] = (uint16_t)f32_to_bf16((0.0f + v) + r);
      } else {
        reinterpret_cast<float*>(out)[o] = v;
      }
    }
  }
}

// m <= 32: one chunk of 16 (MT = 1) or 32 (MT = 2) rows.
template <int NT, int EPI, int WAVES, int UNROLL>
void launch_variant(const uint16_t* xt, const uint16_t* w, uint32_t m, uint32_t n, uint32_t k, uint32_t splits,
                    const uint16_t* residual, void* out, uint32_t ldo, uint32_t* err, hipStream_t s) {
  const uint32_t kb = k / 32;
  const uint32_t kb_split = (kb + splits - 1) / splits;
  const uint32_t x_mtiles = act_mtiles(m);
  dim3 grid(n / (16 * NT), splits, 1);
  if (m <= 16)
    hipLaunchKernelGGL((gemm_kernel<NT, 1, EPI, WAVES, UNROLL>), grid, dim3(WAVES * 64), 0, s, xt, w, m, kb, kb_split,
                       x_mtiles, residual, out, ldo, err, RowNormArgs{});
  else
    hipLaunchKernelGGL((gemm_kernel<NT, 2, EPI, WAVES, UNROLL>), grid, dim3(WAVES * 64), 0, s, xt, w, m, kb, kb_split,
                       x_mtiles, residual, out, ldo, err, RowNormArgs{});
}

// 32 < m <= 256 (a speculative verify, a small prefill chunk): one split, the
// rows in chunks of 64 (MT = 4, unroll 2) or 32 (MT = 2, unroll 4). The
// 64-row chunk halves how often each weight tile is fetched; with 8 waves its
// wave-partial buffer is 128 KiB of LDS (one workgroup per CU), so it is
// taken there only when the launch fits in one round of the 256 CUs.
// Measured at 160 rows (8B shapes, cold weights, us per launch):
//   QKV 6144 x 4096    NT 4, 8 waves: 32-row 29.9, 64-row 38.1 (288 workgroups)
//   O 4096 x 4096      NT 4, 8 waves: 32-row 28.3, 64-row 20.2
//   down 4096 x 12288  NT 4, 8 waves: 32-row 78.5, 64-row 55.5
//   gate/up 24576      64-row: NT 4 with 4 waves 94.2, NT 2 112.6 (32-row NT 2: 128.4)
//   LM head 151936     NT 4, 4 waves: 32-row 788, 64-row 618
// Also slower on every shape: unroll 1, 2-wave workgroups, 128-row chunks
// (gate/up 96 against 106-147, down 56 against 58-95).
template <int NT, int EPI, int WAVES>
void launch_wide(const uint16_t* xt, const uint16_t* w, uint32_t m, uint32_t n, uint32_t k, const uint16_t* residual,
                 void* out, uint32_t ldo, uint32_t* err, hipStream_t s) {
  const uint32_t kb = k / 32;
  const uint32_t x_mtiles = act_mtiles(m);
  const uint32_t slices = n / (16 * NT);
  if (WAVES == 8 && slices * ((m + 63) / 64) > 256) {
    dim3 grid(slices, 1, (m + 31) / 32);
    hipLaunchKernelGGL((gemm_kernel<NT, 2, EPI, WAVES, 4>), grid, dim3(WAVES * 64), 0, s, xt, w, m, kb, kb, x_mtiles,
                       residual, out, ldo, err, RowNormArgs{});
  } else {
    dim3 grid(slices, 1, (m + 63) / 64);
    hipLaunchKernelGGL((gemm_kernel<NT, 4, EPI, WAVES, 2>), grid, dim3(WAVES * 64), 0, s, xt, w, m, kb, kb, x_mtiles,
                       residual, out, ldo, err, RowNormArgs{});
  }
}

// 32 < m <= 256 rows, n % 128 == 0 (a speculative verify; the epilogues a
// wide batch's projections use): the activation panel of each k-block is
// staged in LDS once per workgroup and shared by its 4 waves; each wave
// streams its own 2 weight tiles per k-block into a register ring. The
// launches above read the activations once per 64 weight rows from L2 and
// the weights once per row chunk; here each workgroup reads the activations
// once per 128 weight rows and each weight tile once. Split-K across
// workgroups (FH_EPI_PARTIAL) fills the CUs for the narrow projections; the
// consumer adds the slabs in split order.
//
// MT: 16-row activation tiles computed (even, >= ceil(m / 16)). Per k-block
// a wave issues its 2 weight tiles (register loads, LW = 6 k-blocks ahead)
// and its share of the panel (XPW direct-to-LDS tile loads, LX k-blocks
// ahead; the share is uniform, spare loads refetch tile MT - 1 into spare
// slots). Direct-to-LDS loads and register loads complete out of order with
// respect to each other (only loads of one kind complete in issue order), so
// the wait before k-block kb is per kind: if W(kb) were outstanding, so
// would be the 2 (LW - 1) weight loads after it; if the panel of kb were,
// the XPW (LX - 1) panel loads after it. Waiting until at most the smaller
// of the two counts is outstanding covers both. LX is sized per XPW so that
// the weight count (10) is the smaller one and the weight stream keeps 5
// k-blocks in flight; with a single count over both kinds (the loads of
// one k-block assumed complete once all later ones were) the fast panel
// loads overtook the weight stream and MFMAs read weight registers and
// panel tiles before they arrived. Measured at 160 rows, cold weights, us
// per launch (against the 64/32-row launches above): gate/up 24576 x 4096
// 55 (95), down 4096 x 12288 in 8 splits 28 (56), O 4096 x 4096 in 8 splits
// 14 (20), QKV 6144 x 4096 in 5 splits 18 (30), LM head 151936 x 4096 306
// (617). Weight rings of 4 and 8 k-blocks (gate/up 65, 56), 2 or 8 waves, 4
// weight tiles per wave and 1 per wave were slower.
constexpr int kPanelWaves = 4, kPanelTilesPerWave = 2, kPanelLW = 6;
static_assert(16 * kPanelWaves * kPanelTilesPerWave == kPanelCols, "a workgroup covers kPanelCols weight rows");
constexpr int panel_xpw(int mt) { return (mt + kPanelWaves - 1) / kPanelWaves; }
constexpr int panel_lx(int mt) {
  return 1 + (kPanelTilesPerWave * (kPanelLW - 1) + panel_xpw(mt) - 1) / panel_xpw(mt);
}

constexpr unsigned panel_wait_vm(unsigned n) { return (n & 15u) | ((n >> 4) << 14) | (7u << 4) | (15u << 8); }

template <int B, int E, class F>
__device__ __forceinline__ void panel_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    panel_for<B + 1, E>(f);
  }
}

template <int MT, int EPI>
__global__ __launch_bounds__(kPanelWaves * 64) void gemm_panel_kernel(const uint16_t* __restrict__ xt,
                                                                     const uint16_t* __restrict__ w, uint32_t m,
                                                                     uint32_t x_mtiles, uint32_t kb_count,
                                                                     uint32_t kb_split, void* out, uint32_t ldo,
                                                                     uint32_t* err) {
  constexpr int WAVES = kPanelWaves, NTW = kPanelTilesPerWave, LW = kPanelLW, LX = panel_lx(MT);
  constexpr int XPW = panel_xpw(MT), XT = XPW * WAVES, XST = LX + 1, WSL = LW + 1;
  constexpr int P = LW > LX ? LW : LX;  // prologue steps
  constexpr unsigned kWLater = NTW * (LW - 1), kXLater = XPW * (LX - 1);
  constexpr unsigned kInFlight = kWLater < kXLater ? kWLater : kXLater;
  static_assert(kInFlight < 64 && kInFlight >= kWLater, "the weight stream keeps LW - 1 k-blocks in flight");
  __shared__ __attribute__((aligned(16))) u32x4 panel[XST][XT][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t slice = blockIdx.x, split = blockIdx.y;
  const uint32_t kb_lo = split * kb_split;
  // A split past the end of k (ceil rounding) writes zero partials.
  const uint32_t nkb = kb_lo < kb_count ? min(kb_split, kb_count - kb_lo) : 0u;
  const uint32_t tile0 = (slice * WAVES + wave) * NTW;

  f32x4 acc[NTW][MT];
#pragma unroll
  for (int t = 0; t < NTW; ++t)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[t][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (nkb > 0) {
    const uint32_t last = nkb - 1;
    // Workgroups start their k-range at staggered k-blocks (and wrap), so
    // the grid's concurrent weight loads spread over the HBM channels. The
    // order depends on the launch coordinates only, not on m.
    const uint32_t rot = (slice * 7u + split * 5u) % nkb;
    // k-block of step i; steps past the end repeat the last k-block, so the
    // count of loads in flight is the same at every step.
    auto kmap = [&](uint32_t i) -> uint64_t {
      uint32_t j = min(i, last) + rot;
      if (j >= nkb) j -= nkb;
      return kb_lo + j;
    };
    const u32x4* wp = reinterpret_cast<const u32x4*>(w) + (uint64_t)tile0 * kb_count * 64 + lane;
    const uint64_t w_tile = (uint64_t)kb_count * 64;
    const u32x4* xp = reinterpret_cast<const u32x4*>(xt) + lane;
    const uint64_t x_kb = (uint64_t)x_mtiles * 64;
    u32x4 wr[WSL][NTW];
    auto load_w = [&](auto slot_c, uint32_t i) {
      const uint64_t k = kmap(i);
#pragma unroll
      for (int t = 0; t < NTW; ++t)
        wr[decltype(slot_c)::value][t] = __builtin_nontemporal_load(wp + t * w_tile + k * 64);
    };
    auto fetch_x = [&](uint32_t i) {
      const uint64_t k = kmap(i);
      const uint32_t st = i % XST;
#pragma unroll
      for (int t = 0; t < XPW; ++t) {
        const int j = wave + t * WAVES;
        const int src = j < MT ? j : MT - 1;
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(xp + k * x_kb + src * 64),
                                         (__attribute__((address_space(3))) void*)&panel[st][j][0], 16, 0, 0);
      }
    };
    // Prologue: W(0 .. LW - 1) and panels 0 .. LX - 1.
    panel_for<0, P>([&](auto j_c) {
      constexpr int j = decltype(j_c)::value - P;
      if constexpr (j + LW >= 0) load_w(std::integral_constant<int, (j + LW) % WSL>{}, j + LW);
      if constexpr (j + LX >= 0) fetch_x(j + LX);
    });
    auto step = [&](auto s_c, uint32_t kb) {
      constexpr int S = decltype(s_c)::value;
      __builtin_amdgcn_s_waitcnt(panel_wait_vm(kInFlight));
      // Every wave's share of panel kb is in LDS, and every wave is done
      // reading panel kb - 1, whose stage the next fetch overwrites.
      __builtin_amdgcn_s_barrier();
      load_w(std::integral_constant<int, (S + LW) % WSL>{}, kb + LW);
      fetch_x(kb + LX);
      const uint32_t st = kb % XST;
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const u32x4 xv = panel[st][j][lane];
#pragma unroll
        for (int t = 0; t < NTW; ++t)
          acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(wr[S][t]), as_b8(xv), acc[t][j], 0, 0, 0);
      }
    };
    uint32_t kb = 0;
    for (; kb + WSL <= nkb; kb += WSL) panel_for<0, WSL>([&](auto s_c) { step(s_c, kb + decltype(s_c)::value); });
    panel_for<0, WSL - 1>([&](auto s_c) {
      if (kb + decltype(s_c)::value < nkb) step(s_c, kb + decltype(s_c)::value);
    });
    __builtin_amdgcn_s_waitcnt(panel_wait_vm(0));  // the repeated loads past the end
  }

  // D layout: lane l, element e holds weight row n = 16 nt + 4 (l / 16) + e
  // and activation row m = 16 mt + l % 16.
  const uint32_t q = lane >> 4, c = lane & 15;
  if constexpr (EPI == FH_EPI_SWIGLU) {
    bool bad = false;
#pragma unroll
    for (int p = 0; p < NTW / 2; ++p) {
      const uint32_t col = ((tile0 + 2 * p) / 2) * 16 + 4 * q;  // first of 4 output columns
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const uint32_t row = j * 16 + c;
        if (row >= m) continue;
        uint32_t y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          y[e] = swiglu_bf16(round_bf16(acc[2 * p][j][e]), round_bf16(acc[2 * p + 1][j][e]), bad);
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + act_offset_m(row, col, act_mtiles(m))) =
            make_uint2(y[0] | (y[1] << 16), y[2] | (y[3] << 16));
      }
    }
    if (bad) raise_error(err, ERR_NONFINITE);
  } else {
    static_assert(EPI == FH_EPI_PARTIAL || EPI == FH_EPI_F32, "panel epilogues");
    float* o = reinterpret_cast<float*>(out) + (EPI == FH_EPI_PARTIAL ? (uint64_t)split * kPanelRows * ldo : 0u);
#pragma unroll
    for (int t = 0; t < NTW; ++t) {
      const uint32_t n = (tile0 + t) * 16 + 4 * q;
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const uint32_t row = j * 16 + c;
        if (row < m) *reinterpret_cast<f32x4*>(o + (uint64_t)row * ldo + n) = acc[t][j];
      }
    }
  }
}

template <int EPI>
void launch_panel(const uint16_t* xt, const uint16_t* w, uint32_t m, uint32_t n, uint32_t k, uint32_t splits,
                  void* out, uint32_t ldo, uint32_t* err, hipStream_t s) {
  const uint32_t kb = k / 32;
  const uint32_t kb_split = (kb + splits - 1) / splits;
  const dim3 grid(n / kPanelCols, splits);
  uint32_t mt = (m + 15) / 16;
  mt += mt & 1u;
#define FH_PANEL(MT_)                                                                                        \
  hipLaunchKernelGGL((gemm_panel_kernel<MT_, EPI>), grid, dim3(kPanelWaves * 64), 0, s, xt, w, m, act_mtiles(m), \
                     kb, kb_split, out, ldo, err)
  switch (mt) {
    case 4: FH_PANEL(4); break;
    case 6: FH_PANEL(6); break;
    case 8: FH_PANEL(8); break;
    case 10: FH_PANEL(10); break;
    case 12: FH_PANEL(12); break;
    case 14: FH_PANEL(14); break;
    default: FH_PANEL(16); break;
  }
#undef FH_PANEL
}

// Shape policy (measured on MI355X at m = 32, cold weights). Weights of up
// to 16K rows take the most n-tiles per wave (4, 2, 1) that still give
// 256 workgroups with the caller's splits (4 keeps the activation traffic
// at half the weight traffic), or NT = 3 for split-K partials when only
// that fills the CUs (the 8B QKV weight); the smallest (2 for SwiGLU pairs)
// when none does. A wave walks at least 4 k-blocks: 8 waves when a split
// holds 32 k-blocks or more, else 4. The 8B projections keep NT = 4 (3 for
// QKV) with 8 waves; the Qwen3-0.6B ones, too small to fill the CUs with 4,
// went (us per launch, 32 rows) from QKV 6.2 to 4.1 (NT 2, 4 waves), O 6.0
// to 3.3-4.2 (NT 1), gate/up 6.7 to 5.1 (NT 2, 8 waves), down 6.1 to 4.2
// (NT 1). The fused 8B gate/up weight (24K rows) keeps NT = 2 with 4 waves,
// twice as many workgroups in flight (NT = 4 with 4 waves, half the
// activation traffic: 1.41 -> 1.54 ms per step at 32 rows, 1.26 -> 1.42 at
// one row); the LM head (152K rows) has n-tiles
// enough for NT = 4 with 4 waves (NT = 2 at up to 16 rows).
// The weight-streaming variant (n-tiles per wave, waves) launch_epi takes for
// m <= 32 rows; {0, 0} where it has none.
struct SmallVariant {
  uint32_t nt, waves;
};

SmallVariant small_variant(uint32_t epi, uint32_t m, uint32_t n, uint32_t k, uint32_t splits) {
  const bool swiglu = epi == FH_EPI_SWIGLU;
  // Three n-tiles per wave where that puts exactly one workgroup on each of
  // the 256 CUs and four would leave some idle (the 8B QKV weight: 6144 rows
  // in 2 splits, 192 -> 256 workgroups, 11.4 -> 10.8 us).
  if (epi == FH_EPI_PARTIAL && n % 48 == 0 && n / 48 * splits == 256 && (n % 64 != 0 || n / 64 * splits < 256))
    return {3, 8};
  if (n < 16384) {
    const uint32_t waves = (k / 32 + splits - 1) / splits >= 32 ? 8 : 4;
    auto fills = [&](uint32_t nt) { return n % (16 * nt) == 0 && n / (16 * nt) * splits >= 256; };
    if (fills(4)) return {4, waves};
    if (n % 32 == 0 && (fills(2) || swiglu)) return {2, waves};
    return swiglu ? SmallVariant{0, 0} : SmallVariant{1, waves};
  }
  // One row (the gate/up weight and the LM head): 2 n-tiles per wave with 8
  // waves per workgroup, half as many workgroups as with 4 waves for the
  // same waves in flight. Each of them runs the row's residual + RMSNorm in
  // its prologue (launch_gemm_rownorm) and reads the row and its split-K
  // slabs to do so: 8B batch 1, 3.268 -> 3.244 ms device time per step
  // (gate/up -20 us, head -4 us; alternating runs).
  if (m == 1 && n % 32 == 0) return {2, 8};
  // The LM head: at up to 16 rows (one activation tile) 2 n-tiles per wave
  // read its 1.24 GB in 182 us instead of 191 (8B, batch 1); at 32 rows 4.
  if (!swiglu && n % 64 == 0) return {m <= 16 ? 2u : 4u, 4};
  if (n % 32 == 0) return {2, 4};
  return swiglu ? SmallVariant{0, 0} : SmallVariant{1, 4};
}

// Shape policy (measured on MI355X at m = 32, cold weights). Weights of up
// to 16K rows take the most n-tiles per wave (4, 2, 1) that still give
// 256 workgroups with the caller's splits (4 keeps the activation traffic
// at half the weight traffic), or NT = 3 for split-K partials when only
// that fills the CUs (the 8B QKV weight); the smallest (2 for SwiGLU pairs)
// when none does. A wave walks at least 4 k-blocks: 8 waves when a split
// holds 32 k-blocks or more, else 4. The 8B projections keep NT = 4 (3 for
// QKV) with 8 waves; the Qwen3-0.6B ones, too small to fill the CUs with 4,
// went (us per launch, 32 rows) from QKV 6.2 to 4.1 (NT 2, 4 waves), O 6.0
// to 3.3-4.2 (NT 1), gate/up 6.7 to 5.1 (NT 2, 8 waves), down 6.1 to 4.2
// (NT 1). The fused 8B gate/up weight (24K rows) keeps NT = 2 with 4 waves,
// twice as many workgroups in flight (NT = 4 with 4 waves, half the
// activation traffic: 1.41 -> 1.54 ms per step at 32 rows, 1.26 -> 1.42 at
// one row); the LM head (152K rows) has n-tiles
// enough for NT = 4 with 4 waves (NT = 2 at up to 16 rows).
template <int EPI>
void launch_epi(const uint16_t* xt, const uint16_t* w, uint32_t m, uint32_t n, uint32_t k, uint32_t splits,
                const uint16_t* residual, void* out, uint32_t ldo, uint32_t* err, hipStream_t s) {
  if constexpr (EPI == FH_EPI_PARTIAL || EPI == FH_EPI_SWIGLU || EPI == FH_EPI_F32) {
    if (m > kMaxRows && m <= kPanelRows && n % kPanelCols == 0) {
      launch_panel<EPI>(xt, w, m, n, k, splits, out, ldo, err, s);
      return;
    }
  }
  if constexpr (EPI != FH_EPI_PARTIAL) {
    if (m > kMaxRows) {
      if (n % 64 == 0 && n < 16384 && EPI != FH_EPI_SWIGLU)
        launch_wide<4, EPI, 8>(xt, w, m, n, k, residual, out, ldo, err, s);
      else if (n % 64 == 0)
        launch_wide<4, EPI, 4>(xt, w, m, n, k, residual, out, ldo, err, s);
      else if (n % 32 == 0)
        launch_wide<2, EPI, 4>(xt, w, m, n, k, residual, out, ldo, err, s);
      else if constexpr (EPI != FH_EPI_SWIGLU)
        launch_wide<1, EPI, 4>(xt, w, m, n, k, residual, out, ldo, err, s);
      return;
    }
  }
  const SmallVariant v = small_variant(EPI, m, n, k, splits);
#define FH_VARIANT(NT_, WAVES_) launch_variant<NT_, EPI, WAVES_, 4>(xt, w, m, n, k, splits, residual, out, ldo, err, s)
  if (v.nt == 4) {
    if (v.waves == 8) FH_VARIANT(4, 8); else FH_VARIANT(4, 4);
  } else if (v.nt == 2) {
    if (v.waves == 8) FH_VARIANT(2, 8); else FH_VARIANT(2, 4);
  } else if constexpr (EPI != FH_EPI_SWIGLU) {
    if (v.nt == 3) {
      if constexpr (EPI == FH_EPI_PARTIAL) FH_VARIANT(3, 8);
    } else if (v.nt == 1) {
      if (v.waves == 8) FH_VARIANT(1, 8); else FH_VARIANT(1, 4);
    }
  }
#undef FH_VARIANT
}

// One row with its residual + RMSNorm in the prologue (launch_gemm_rownorm):
// the grid and kernel of launch_variant for m = 1, x from the norm.
template <int NT, int EPI, int WAVES, int NS, int NJ>
void launch_rownorm_variant(const uint16_t* w, uint32_t n, uint32_t k, uint32_t splits, const RowNormArgs& na,
                            void* out, uint32_t ldo, uint32_t* err, hipStream_t s) {
  const uint32_t kb = k / 32;
  const uint32_t kb_split = (kb + splits - 1) / splits;
  hipLaunchKernelGGL((gemm_kernel<NT, 1, EPI, WAVES, 4, NS, NJ>), dim3(n / (16 * NT), splits, 1), dim3(WAVES * 64), 0,
                     s, nullptr, w, 1u, kb, kb_split, 1u, nullptr, out, ldo, err, na);
}

template <int EPI, int NS, int NJ>
bool launch_rownorm_ns(SmallVariant v, const uint16_t* w, uint32_t n, uint32_t k, uint32_t splits,
                       const RowNormArgs& na, void* out, uint32_t ldo, uint32_t* err, hipStream_t s, bool dry) {
  // The one-row shapes of the Qwen3 projections: QKV (PARTIAL) NT 3 with 8
  // waves (8B) or NT 2 with 4 (0.6B); gate/up (SWIGLU) and the LM head (F32)
  // NT 2 with 8 waves (NT 2 with 4 kept for narrower shapes).
  if constexpr (EPI == FH_EPI_PARTIAL) {
    if (v.nt == 3 && v.waves == 8) {
      if (!dry) launch_rownorm_variant<3, EPI, 8, NS, NJ>(w, n, k, splits, na, out, ldo, err, s);
      return true;
    }
  }
  if constexpr (EPI == FH_EPI_SWIGLU || EPI == FH_EPI_F32) {
    if (v.nt == 2 && v.waves == 8) {
      if (!dry) launch_rownorm_variant<2, EPI, 8, NS, NJ>(w, n, k, splits, na, out, ldo, err, s);
      return true;
    }
  }
  if (v.nt == 2 && v.waves == 4) {
    if (!dry) launch_rownorm_variant<2, EPI, 4, NS, NJ>(w, n, k, splits, na, out, ldo, err, s);
    return true;
  }
  return false;
}

template <int EPI, int NJ>
bool launch_rownorm_epi(SmallVariant v, const uint16_t* w, uint32_t n, uint32_t k, uint32_t splits,
                        const RowNormArgs& na, void* out, uint32_t ldo, uint32_t* err, hipStream_t s, bool dry) {
  switch (na.splits) {
    case 0:
      if constexpr (EPI == FH_EPI_PARTIAL) return launch_rownorm_ns<EPI, 0, NJ>(v, w, n, k, splits, na, out, ldo, err, s, dry);
      return false;
    case 4: return launch_rownorm_ns<EPI, 4, NJ>(v, w, n, k, splits, na, out, ldo, err, s, dry);
    case 6: return launch_rownorm_ns<EPI, 6, NJ>(v, w, n, k, splits, na, out, ldo, err, s, dry);
    default: return false;
  }
}

bool rownorm_dispatch(const uint16_t* w, uint32_t n, uint32_t k, uint32_t epilogue, uint32_t splits,
                      const RowNormArgs& na, void* out, uint32_t ldo, uint32_t* err, hipStream_t s, bool dry) {
  if (splits == 0 || k % 256 != 0 || k < 1024 || k > 4096 || (epilogue != FH_EPI_PARTIAL && splits != 1))
    return false;
  const SmallVariant v = small_variant(epilogue, 1, n, k, splits);
  const bool two = k / 8 > kRowNormThreads;
  switch (epilogue) {
    case FH_EPI_PARTIAL:
      return two ? launch_rownorm_epi<FH_EPI_PARTIAL, 2>(v, w, n, k, splits, na, out, ldo, err, s, dry)
                 : launch_rownorm_epi<FH_EPI_PARTIAL, 1>(v, w, n, k, splits, na, out, ldo, err, s, dry);
    case FH_EPI_SWIGLU:
      return two ? launch_rownorm_epi<FH_EPI_SWIGLU, 2>(v, w, n, k, splits, na, out, ldo, err, s, dry)
                 : launch_rownorm_epi<FH_EPI_SWIGLU, 1>(v, w, n, k, splits, na, out, ldo, err, s, dry);
    case FH_EPI_F32:
      return two ? launch_rownorm_epi<FH_EPI_F32, 2>(v, w, n, k, splits, na, out, ldo, err, s, dry)
                 : launch_rownorm_epi<FH_EPI_F32, 1>(v, w, n, k, splits, na, out, ldo, err, s, dry);
    default: return false;
  }
}

// Splits so that a launch has about 256 workgroups (one per CU), each split
// keeping at least 16 k-blocks.
uint32_t choose_splits(uint32_t n, uint32_t k) {
  const uint32_t groups = n % 64 == 0 && n < 16384 ? n / 64 : n % 32 == 0 ? n / 32 : n / 16;
  const uint32_t kb = k / 32;
  uint32_t s = 256 / groups;
  const uint32_t max_s = kb / 16 > 0 ? kb / 16 : 1;
  if (s > max_s) s = max_s;
  if (s < 1) s = 1;
  return s;
}

}  // namespace

uint32_t gemm_default_splits(uint32_t n, uint32_t k) { return choose_splits(n, k); }

// 33..256 rows: about 256 workgroups of 128 weight rows, each split keeping
// at least 16 k-blocks (8B shapes: QKV 5, O 8, down 8, gate/up 1).
uint32_t gemm_panel_splits(uint32_t n, uint32_t k) {
  const uint32_t slices = n / kPanelCols, kb = k / 32;
  uint32_t s = slices ? 256 / slices : 1;
  const uint32_t max_s = kb / 16 > 0 ? kb / 16 : 1;
  if (s > max_s) s = max_s;
  return s < 1 ? 1 : s;
}

bool gemm_rownorm_supported(uint32_t n, uint32_t k, uint32_t epilogue, uint32_t splits, uint32_t norm_splits) {
  RowNormArgs na{};
  na.splits = norm_splits;
  return rownorm_dispatch(nullptr, n, k, epilogue, splits, na, nullptr, 0, nullptr, nullptr, true);
}

hipError_t launch_gemm_rownorm(const uint16_t* w_tiled, uint32_t n, uint32_t k, uint32_t epilogue, uint32_t splits,
                               const RowNormArgs& na, void* out, uint32_t ldo, uint32_t* err, hipStream_t s) {
  if (na.splits > 0 && na.hidden_out == na.hidden_in) return hipErrorInvalidValue;
  if (!rownorm_dispatch(w_tiled, n, k, epilogue, splits, na, out, ldo, err, s, false)) return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_gemm(const uint16_t* x_tiled, const uint16_t* w_tiled, uint32_t m, uint32_t n, uint32_t k,
                       uint32_t epilogue, uint32_t splits, const uint16_t* residual, void* out, uint32_t ldo,
                       uint32_t* err, hipStream_t s) {
  if (splits == 0) return hipErrorInvalidValue;
  if (m > kMaxRows && (epilogue == FH_EPI_PARTIAL ? !gemm_partial_rows_ok(m, n) : splits != 1))
    return hipErrorInvalidValue;
  switch (epilogue) {
    case FH_EPI_BF16: launch_epi<FH_EPI_BF16>(x_tiled, w_tiled, m, n, k, 1, residual, out, ldo, err, s); break;
    case FH_EPI_RESIDUAL: launch_epi<FH_EPI_RESIDUAL>(x_tiled, w_tiled, m, n, k, 1, residual, out, ldo, err, s); break;
    case FH_EPI_SWIGLU: launch_epi<FH_EPI_SWIGLU>(x_tiled, w_tiled, m, n, k, 1, residual, out, ldo, err, s); break;
    case FH_EPI_F32: launch_epi<FH_EPI_F32>(x_tiled, w_tiled, m, n, k, 1, residual, out, ldo, err, s); break;
    case FH_EPI_PARTIAL: launch_epi<FH_EPI_PARTIAL>(x_tiled, w_tiled, m, n, k, splits, residual, out, ldo, err, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace fh
