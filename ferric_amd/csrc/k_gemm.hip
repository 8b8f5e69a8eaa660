// K1 projections for decode (m <= 32 token rows): weight-streaming GEMM on
// gfx950 MFMA (v_mfma_f32_16x16x32_bf16), FP32 accumulation, fused epilogues.
//
// Data layout: the weight W[n][k] is stored in MFMA tile order (common.hpp
// tiled_offset): each 16x32 tile is one fully coalesced 1 KiB wave load that
// lands directly in the A-operand registers — no LDS staging, no transpose.
// The activation x[m][k] (row-major, small, L2-resident) is the B operand:
// lane l reads 16 contiguous bytes of row (l % 16).
//
// Work split: a workgroup owns NT consecutive 16-row n-tiles over the whole
// reduction; its 8 waves split the k-blocks into 8 contiguous ranges, and the
// 8 partial tiles are added in wave order through LDS (deterministic). The
// epilogue then writes
//   FH_EPI_BF16     out = bf16(acc)                      (Q/K/V, gemm.rs:161 beta = 0)
//   FH_EPI_RESIDUAL out = bf16((0 + acc) + residual)     (O and down + residual,
//                    v5 collective.rs:25-60; gemm.rs:262-336 beta = 1)
//   FH_EPI_SWIGLU   out = swiglu(bf16(gate), bf16(up))   (gate/up + K6 fused;
//                    tiles 2j / 2j+1 are gate / up of the same 16 columns)
//   FH_EPI_F32      out = acc (f32)                      (FP32 LM head, v8 projection.rs:66)
// The rounding points are the reference's (one bf16 RNE per projection; gate
// and up narrowed before SwiGLU); the FP32 summation order is reassociated
// (k-blocks of 32 per MFMA, 8 wave ranges), as the reference's own wave and
// MFMA profiles reassociate (v5 projection.rs:15, :241).
#include "common.hpp"
#include "kernels.hpp"
#include "../../include/ferric_hip.h"

namespace fh {

namespace {

constexpr int kWaves = 8;
constexpr int kGemmThreads = kWaves * 64;
constexpr int kUnroll = 4;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8 as_b8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

template <int NT, int MT, int EPI>
__global__ __launch_bounds__(kGemmThreads) void gemm_skinny_kernel(const uint16_t* __restrict__ x, uint32_t ldx,
                                                                   const uint16_t* __restrict__ w, uint32_t m,
                                                                   uint32_t kb_count,
                                                                   const uint16_t* residual, void* out,
                                                                   uint32_t ldo) {
  __shared__ float red[kWaves][NT * MT * 256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t tile0 = blockIdx.x * NT;
  const uint32_t kb_lo = (kb_count * wave) / kWaves;
  const uint32_t kb_hi = (kb_count * (wave + 1)) / kWaves;

  const u32x4* wp[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
    wp[nt] = reinterpret_cast<const u32x4*>(w) + ((uint64_t)(tile0 + nt) * kb_count + kb_lo) * 64 + lane;
  const u32x4* xp[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    uint32_t row = mt * 16 + (lane & 15);
    if (row >= m) row = m - 1;  // rows past m feed columns that are never stored
    xp[mt] = reinterpret_cast<const u32x4*>(x + (uint64_t)row * ldx + kb_lo * 32 + (lane >> 4) * 8);
  }

  f32x4 acc[NT][MT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const uint32_t steps = kb_hi - kb_lo;
  uint32_t s = 0;
  for (; s + kUnroll <= steps; s += kUnroll) {
    u32x4 wv[kUnroll][NT], xv[kUnroll][MT];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) wv[u][nt] = __builtin_nontemporal_load(wp[nt] + (uint64_t)(s + u) * 64);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) xv[u][mt] = xp[mt][(s + u) * 4];
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(wv[u][nt]), as_b8(xv[u][mt]), acc[nt][mt], 0, 0, 0);
  }
  for (; s < steps; ++s) {
    u32x4 wv[NT], xv[MT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) wv[nt] = __builtin_nontemporal_load(wp[nt] + (uint64_t)s * 64);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xv[mt] = xp[mt][s * 4];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(wv[nt]), as_b8(xv[mt]), acc[nt][mt], 0, 0, 0);
  }

  // D layout of the 16x16 MFMA: lane l, element e holds row i = 4*(l/16) + e
  // (the weight row n) and column j = l % 16 (the activation row m). Store
  // transposed as [j][i] so the epilogue walks n fastest (coalesced stores).
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        red[wave][(nt * MT + mt) * 256 + (lane & 15) * 16 + 4 * (lane >> 4) + e] = acc[nt][mt][e];
  __syncthreads();

  if constexpr (EPI == FH_EPI_SWIGLU) {
    static_assert(NT == 2, "SwiGLU epilogue pairs a gate tile with an up tile");
    bool bad = false;
    for (int idx = threadIdx.x; idx < MT * 256; idx += kGemmThreads) {
      const int mt = idx >> 8, j = (idx >> 4) & 15, i = idx & 15;
      const uint32_t row = mt * 16 + j;
      float g = red[0][(0 * MT + mt) * 256 + j * 16 + i];
      float u = red[0][(1 * MT + mt) * 256 + j * 16 + i];
#pragma unroll
      for (int wv = 1; wv < kWaves; ++wv) {
        g += red[wv][(0 * MT + mt) * 256 + j * 16 + i];
        u += red[wv][(1 * MT + mt) * 256 + j * 16 + i];
      }
      if (row < m) {
        uint32_t y = swiglu_bf16(round_bf16(g), round_bf16(u), bad);
        reinterpret_cast<uint16_t*>(out)[(uint64_t)row * ldo + blockIdx.x * 16 + i] = (uint16_t)y;
      }
    }
    (void)bad;  // nonfinite activations surface at the next norm / the logits
  } else {
    for (int idx = threadIdx.x; idx < NT * MT * 256; idx += kGemmThreads) {
      const int tm = idx >> 8, j = (idx >> 4) & 15, i = idx & 15;
      const int nt = tm / MT, mt = tm % MT;
      const uint32_t row = mt * 16 + j;
      float v = red[0][idx];
#pragma unroll
      for (int wv = 1; wv < kWaves; ++wv) v += red[wv][idx];
      if (row >= m) continue;
      const uint64_t n = (uint64_t)(tile0 + nt) * 16 + i;
      const uint64_t o = (uint64_t)row * ldo + n;
      if constexpr (EPI == FH_EPI_BF16) {
        reinterpret_cast<uint16_t*>(out)[o] = (uint16_t)f32_to_bf16(v);
      } else if constexpr (EPI == FH_EPI_RESIDUAL) {
        float r = bf16_to_f32(residual[o]);
        reinterpret_cast<uint16_t*>(out)[o] = (uint16_t)f32_to_bf16((0.0f + v) + r);
      } else {
        reinterpret_cast<float*>(out)[o] = v;
      }
    }
  }
}

template <int NT, int EPI>
hipError_t launch_nt(const uint16_t* x, uint32_t ldx, const uint16_t* w, uint32_t m, uint32_t n, uint32_t k,
                     const uint16_t* residual, void* out, uint32_t ldo, hipStream_t s) {
  dim3 grid(n / (16 * NT));
  if (m <= 16)
    hipLaunchKernelGGL((gemm_skinny_kernel<NT, 1, EPI>), grid, dim3(kGemmThreads), 0, s, x, ldx, w, m, k / 32, residual,
                       out, ldo);
  else
    hipLaunchKernelGGL((gemm_skinny_kernel<NT, 2, EPI>), grid, dim3(kGemmThreads), 0, s, x, ldx, w, m, k / 32, residual,
                       out, ldo);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(const uint16_t* x, uint32_t ldx, const uint16_t* w_tiled, uint32_t m, uint32_t n, uint32_t k,
                       uint32_t epilogue, const uint16_t* residual, void* out, uint32_t ldo, hipStream_t s) {
  switch (epilogue) {
    case FH_EPI_BF16:
      return launch_nt<1, FH_EPI_BF16>(x, ldx, w_tiled, m, n, k, residual, out, ldo, s);
    case FH_EPI_RESIDUAL:
      return launch_nt<1, FH_EPI_RESIDUAL>(x, ldx, w_tiled, m, n, k, residual, out, ldo, s);
    case FH_EPI_SWIGLU:
      return launch_nt<2, FH_EPI_SWIGLU>(x, ldx, w_tiled, m, n, k, residual, out, ldo, s);
    case FH_EPI_F32:
      return launch_nt<1, FH_EPI_F32>(x, ldx, w_tiled, m, n, k, residual, out, ldo, s);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace fh
