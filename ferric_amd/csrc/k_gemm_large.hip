// K1 projections for prefill and wide verify batches (m > 32 token rows):
// bf16 MFMA (v_mfma_f32_16x16x32_bf16), FP32 accumulation, compute-bound.
//
// Operands come from their tile orders (common.hpp): the weight in weight
// tile order and the activation in activation tile order with act_mtiles(m)
// row tiles, so every operand fetch of a wave is one contiguous 1 KiB in the
// exact MFMA register layout. Two kernels:
//  * gemm_large_xd_kernel (n % 256 == 0: every projection): 256 x 256
//    blocks of 8 waves sharing each k-block's weight tiles through LDS,
//    activation tiles loaded by each wave;
//  * gemm_large_kernel (the LM head's 151936 rows): 128 x 128 blocks of 4
//    waves loading operands straight into registers (each tile fetched by
//    two waves; the second fetch hits the CU's cache).
// Each wave accumulates its MFMA tiles over the whole k range.
//
// Epilogues (same rounding points as the decode kernel, no split-K here):
//   FH_EPI_BF16     out[m][n] = bf16(acc)
//   FH_EPI_RESIDUAL out[m][n] = bf16((0 + acc) + residual[m][n]) (may alias out)
//   FH_EPI_SWIGLU   act = swiglu(bf16(gate), bf16(up)) in activation tile order
//                   (gate/up tiles interleaved by the weight layout)
//   FH_EPI_F32      out[m][n] = acc (FP32 logits)
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"
#include "../../include/ferric_hip.h"

namespace fh {

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kStreamedRows = 256;
constexpr int kNT = 4;  // n-tiles per wave
constexpr int kMT = 4;  // m-tiles per wave
constexpr int kBlockTiles = 2 * kNT;  // 16-row tiles per block side (128 rows)
static_assert(kLargeBlockRows % (16 * 2 * kMT) == 0, "padded rows cover whole blocks");

__device__ __forceinline__ bf16x8 b8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

template <int EPI>
__global__ __launch_bounds__(256) void gemm_large_kernel(const uint16_t* __restrict__ xt,
                                                         const uint16_t* __restrict__ w, uint32_t m,
                                                         uint32_t mtiles, uint32_t kb_count,
                                                         const uint16_t* residual, void* out, uint32_t ldo,
                                                         uint32_t out_mtiles, uint32_t* err) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t nt0 = blockIdx.x * kBlockTiles + (wave & 1) * kNT;  // first 16-row weight tile
  const uint32_t mt0 = blockIdx.y * kBlockTiles + (wave >> 1) * kMT;  // first 16-row activation tile
  if (mt0 * 16 >= m) return;  // this wave's rows are all padding

  // Per k-block: weight tile (nb, kb) at (nb * kb_count + kb) KiB; activation
  // tile (kb, mt) at (kb * mtiles + mt) KiB. Pointers are in 16-byte units.
  const u32x4* wp = reinterpret_cast<const u32x4*>(w) + (uint64_t)nt0 * kb_count * 64 + lane;
  const u32x4* xp = reinterpret_cast<const u32x4*>(xt) + (uint64_t)mt0 * 64 + lane;
  const uint64_t w_tile_stride = (uint64_t)kb_count * 64;  // next n-tile
  const uint64_t x_kb_stride = (uint64_t)mtiles * 64;      // next k-block

  f32x4 acc[kNT][kMT];
#pragma unroll
  for (int i = 0; i < kNT; ++i)
#pragma unroll
    for (int j = 0; j < kMT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 wa[kNT], xa[kMT], wb[kNT], xb[kMT];
  auto load = [&](u32x4(&wv)[kNT], u32x4(&xv)[kMT], uint32_t kb) {
#pragma unroll
    for (int i = 0; i < kNT; ++i) wv[i] = wp[i * w_tile_stride + kb * 64];
#pragma unroll
    for (int j = 0; j < kMT; ++j) xv[j] = xp[kb * x_kb_stride + j * 64];
  };
  auto compute = [&](const u32x4(&wv)[kNT], const u32x4(&xv)[kMT]) {
#pragma unroll
    for (int i = 0; i < kNT; ++i)
#pragma unroll
      for (int j = 0; j < kMT; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b8(wv[i]), b8(xv[j]), acc[i][j], 0, 0, 0);
  };
  load(wa, xa, 0);
  for (uint32_t kb = 0; kb < kb_count; kb += 2) {
    if (kb + 1 < kb_count) load(wb, xb, kb + 1);
    __builtin_amdgcn_sched_barrier(0);
    compute(wa, xa);
    __builtin_amdgcn_sched_barrier(0);
    if (kb + 1 < kb_count) {
      if (kb + 2 < kb_count) load(wa, xa, kb + 2);
      __builtin_amdgcn_sched_barrier(0);
      compute(wb, xb);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // D layout: lane l, element e holds weight row n = 16 nt + 4 (l / 16) + e
  // and activation row m = 16 mt + l % 16.
  const uint32_t q = lane >> 4, c = lane & 15;
  if constexpr (EPI == FH_EPI_SWIGLU) {
    static_assert(kNT % 2 == 0, "gate/up tile pairs");
    bool bad = false;
#pragma unroll
    for (int p = 0; p < kNT / 2; ++p) {
      const uint32_t col = ((nt0 + 2 * p) / 2) * 16 + 4 * q;  // first of 4 output columns
#pragma unroll
      for (int j = 0; j < kMT; ++j) {
        const uint32_t row = (mt0 + j) * 16 + c;
        if (row >= m) continue;
        uint32_t y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          y[e] = swiglu_bf16(round_bf16(acc[2 * p][j][e]), round_bf16(acc[2 * p + 1][j][e]), bad);
        uint2 v = make_uint2(y[0] | (y[1] << 16), y[2] | (y[3] << 16));
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + act_offset_m(row, col, out_mtiles)) = v;
      }
    }
    if (bad) raise_error(err, ERR_NONFINITE);
  } else {
#pragma unroll
    for (int i = 0; i < kNT; ++i) {
      const uint32_t n = (nt0 + i) * 16 + 4 * q;
#pragma unroll
      for (int j = 0; j < kMT; ++j) {
        const uint32_t row = (mt0 + j) * 16 + c;
        if (row >= m) continue;
        const uint64_t o = (uint64_t)row * ldo + n;
        if constexpr (EPI == FH_EPI_F32) {
          *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(out) + o) = acc[i][j];
        } else if constexpr (EPI == FH_EPI_BF16) {
          uint2 v = make_uint2(f32_to_bf16(acc[i][j][0]) | (f32_to_bf16(acc[i][j][1]) << 16),
                               f32_to_bf16(acc[i][j][2]) | (f32_to_bf16(acc[i][j][3]) << 16));
          *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + o) = v;
        } else {
          const uint2 rv = *reinterpret_cast<const uint2*>(residual + o);
          const float r0 = lo_bf16(rv.x), r1 = hi_bf16(rv.x), r2 = lo_bf16(rv.y), r3 = hi_bf16(rv.y);
          uint2 v = make_uint2(f32_to_bf16((0.0f + acc[i][j][0]) + r0) | (f32_to_bf16((0.0f + acc[i][j][1]) + r1) << 16),
                               f32_to_bf16((0.0f + acc[i][j][2]) + r2) | (f32_to_bf16((0.0f + acc[i][j][3]) + r3) << 16));
          *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + o) = v;
        }
      }
    }
  }
}

constexpr int kBigTiles = 16;  // 16-row tiles per block side (256 rows)

// 256 x 256 blocks for weights with n % 256 == 0 (every projection): 8 waves,
// each 8 n-tiles x 4 m-tiles (wave grid 2 along n x 4 along m). Only the
// weight tiles go through LDS: each k-block's 16 weight tiles are fetched
// global -> LDS directly (global_load_lds_dwordx4: lane i's 16 bytes land at
// tile + 16 i, the tile-order layout itself), 2 per wave, into an
// (LW + 1)-stage ring. Every wave loads its own 4 activation tiles straight
// into registers (an (LX + 1)-slot ring; a tile is used by the 2 waves along
// n, so it is fetched twice, the second time from the cache). Per k-block a
// workgroup reads
// 64 KiB out of LDS and writes 16 KiB; sharing the activation tiles through
// LDS as well (96 KiB read, 32 KiB written, the kernel this replaced) made
// LDS the bound, and this form is 14-28 % faster on the 8B projections with
// bit-identical results. Barriers are bare s_barrier: __syncthreads()' fence
// would wait for every load in flight, k-blocks ahead included.
//
// Counters on the gate/up projection (8192 x 24576 x 4096): 100.7M MFMAs of
// 16 cycles keep the MFMA pipe busy 66 % of the kernel's cycles (down 69 %,
// O 58 %, fused QKV 56 %) with no LDS bank conflicts; the library GEMM
// reaches 85 % on the gate/up shape but at a lower clock under the board's
// power limit, about 10 % faster in time.
constexpr unsigned xd_wait_vm(unsigned n) { return (n & 15u) | ((n >> 4) << 14) | (7u << 4) | (15u << 8); }

// Calls f(std::integral_constant<int, I>) for I = B .. E - 1, unrolled at compile time.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// LX / LW: how many k-blocks ahead the activation / weight tiles are
// requested (LW >= LX, so W(kb) is always older than X(kb)). Measured on the
// 8B projections at m = 8192: LX = 3, LW = 4 is 2-7 % faster than 2 / 3
// (212 VGPRs, 80 KiB LDS, still 2 waves per SIMD); deeper rings, reading all
// of a k-block's weight tiles out of LDS up front, and two k-blocks per
// barrier were not faster.
//
// EPI == kEpiQkvRope (the QKV projection of a prefill chunk): a wave's 8
// n-tiles are exactly one head (128 columns) of 64 rows. After the k loop the
// wave stages them in LDS as bf16 rows (the projection's rounding) and lane r
// runs the per-head QK-norm, RoPE and KV append of row r (qk_head.hpp): the
// same lane code and order as the lane-per-head kernel, without the QKV
// output's round trip through HBM or a second launch.
constexpr int kEpiQkvRope = 16;
constexpr int kQkPitch = 68;  // words per staged row: 64 + 4 keeps rows 16-byte aligned, reads conflict-free

template <int EPI, int LX = 3, int LW = 4>
__global__ __launch_bounds__(512) void gemm_large_xd_kernel(const uint16_t* __restrict__ xt,
                                                            const uint16_t* __restrict__ w, uint32_t m,
                                                            uint32_t mtiles, uint32_t kb_count,
                                                            const uint16_t* residual, void* out, uint32_t ldo,
                                                            uint32_t out_mtiles, const QkvRopeArgs qa,
                                                            uint32_t* err) {
  static_assert(LX >= 1 && LW >= LX, "weights requested no later than activations");
  constexpr int WN = 8, WM = 4, WSTAGES = LW + 1, XSLOTS = LX + 1;
  // The wait before k-block kb counts per kind: direct-to-LDS loads (the
  // weight tiles) and register loads (the activation tiles) complete out of
  // order with respect to each other, only loads of one kind in issue order.
  // If W(kb) were outstanding, so would be the 2 (LW - 1) weight loads after
  // it; if X(kb) were, the WM (LX - 1) activation loads after it. At most the
  // smaller count outstanding covers both.
  constexpr unsigned kWLater = 2 * (LW - 1), kXLater = WM * (LX - 1);
  constexpr unsigned kInFlight = kWLater < kXLater ? kWLater : kXLater;
  static_assert(kInFlight < 64, "vmcnt range");
  constexpr size_t kRingBytes = sizeof(u32x4) * WSTAGES * kBigTiles * 64;
  constexpr size_t kStageBytes = EPI == kEpiQkvRope ? 4ull * 8 * 64 * kQkPitch : 0;
  __shared__ __attribute__((aligned(16))) unsigned char lds_raw[kRingBytes > kStageBytes ? kRingBytes : kStageBytes];
  auto& wlds = *reinterpret_cast<u32x4(*)[WSTAGES][kBigTiles][64]>(lds_raw);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Block order by XCD: workgroups go to the 8 XCDs round-robin in dispatch
  // order, so with the plain order each XCD's co-resident workgroups cover
  // 12 n-blocks x 3 m-blocks (8B gate/up) and its L2 holds that many weight
  // and activation k-slices. Here XCD j takes m-blocks j, j + 8, ... four at
  // a time and walks all n-blocks with them: its workgroups cover 4 m x 8 n
  // blocks, fewer distinct operands per k-block (gate/up -4 %, O -8 %, QKV
  // and down unchanged at 8192 rows; outputs identical). Grids whose m-block
  // count is not a multiple of 32 keep the plain order.
  uint32_t gx = blockIdx.x, gy = blockIdx.y;
  if (gridDim.y % 32 == 0) {
    const uint32_t NB = gridDim.x, b = blockIdx.x + NB * blockIdx.y;
    const uint32_t r = b >> 3;  // position within this XCD's share
    const uint32_t group = r / (4 * NB), within = r % (4 * NB);
    gy = (group * 4 + within % 4) * 8 + (b & 7u);
    gx = within / 4;
  }
  const uint32_t bn = gx * kBigTiles, bm = gy * kBigTiles;
  const int wn = wave % 2, wm = wave / 2;
  const uint32_t last = kb_count - 1;
  // The fused QKV epilogue's row lookups (position, page, slot) are
  // requested now and used after the k loop.
  QkvRowSlot row_slot{0u, 0u, false};
  if constexpr (EPI == kEpiQkvRope) {
    const uint32_t row = (bm + wm * 4) * 16 + lane;
    if (row < m) row_slot = qkv_row_slot(row, qa);
  }
  // Weight fetch: tiles 2 wave, 2 wave + 1 of the block.
  const u32x4* wsrc = reinterpret_cast<const u32x4*>(w) + (uint64_t)(bn + 2 * wave) * kb_count * 64 + lane;
  const uint64_t w_tile = (uint64_t)kb_count * 64;
  auto fetch_w = [&](uint32_t kb) {
    const uint32_t k = min(kb, last);
#pragma unroll
    for (int t = 0; t < 2; ++t)
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(wsrc + t * w_tile + (uint64_t)k * 64),
                                       (__attribute__((address_space(3))) void*)&wlds[kb % WSTAGES][2 * wave + t][0],
                                       16, 0, 0);
  };
  // Activation tiles of this wave: (kb, bm + wm * WM + j), into register slot S.
  const u32x4* xsrc = reinterpret_cast<const u32x4*>(xt) + (uint64_t)(bm + wm * WM) * 64 + lane;
  const uint64_t x_kb = (uint64_t)mtiles * 64;
  u32x4 xr[XSLOTS][WM];
  auto load_x = [&](auto slot_c, uint32_t kb) {
    const uint64_t k = min(kb, last);
#pragma unroll
    for (int j = 0; j < WM; ++j) xr[decltype(slot_c)::value][j] = xsrc[k * x_kb + j * 64];
  };

  f32x4 acc[WN][WM];
#pragma unroll
  for (int i = 0; i < WN; ++i)
#pragma unroll
    for (int j = 0; j < WM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Issue order per iteration j: W(j + LW), then X(j + LX); k-blocks past
  // the end are clamped to the last one, so the count of loads in flight is
  // the same at every iteration. The prologue issues in that same order (for
  // LX = 3, LW = 4: W0 W1 X0 W2 X1 W3 X2), so the first iteration's wait
  // covers X0 as well. Issued in another order the compiler adds its own wait for X0
  // inside the loop, and with direct-to-LDS loads in flight that wait is
  // vmcnt(0), draining every load once per loop iteration.
  static_for<0, LW>([&](auto j_c) {
    constexpr int j = decltype(j_c)::value - LW;
    fetch_w(j + LW);
    if constexpr (j + LX >= 0) load_x(std::integral_constant<int, (j + LX) % XSLOTS>{}, j + LX);
  });
  auto step = [&](auto s_c, uint32_t kb) {
    constexpr int S = decltype(s_c)::value;
    __builtin_amdgcn_s_waitcnt(xd_wait_vm(kInFlight));
    __builtin_amdgcn_s_barrier();  // W(kb) of every wave is in LDS
    fetch_w(kb + LW);
    load_x(std::integral_constant<int, (S + LX) % XSLOTS>{}, kb + LX);
    const int st = kb % WSTAGES;
#pragma unroll
    for (int i = 0; i < WN; ++i) {
      const u32x4 wv = wlds[st][wn * WN + i][lane];
#pragma unroll
      for (int j = 0; j < WM; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b8(wv), b8(xr[S][j]), acc[i][j], 0, 0, 0);
    }
  };
  uint32_t kb = 0;
  for (; kb + XSLOTS <= kb_count; kb += XSLOTS)
    static_for<0, XSLOTS>([&](auto s_c) { step(s_c, kb + decltype(s_c)::value); });
  static_for<0, XSLOTS - 1>([&](auto s_c) {
    if (kb + decltype(s_c)::value < kb_count) step(s_c, kb + decltype(s_c)::value);
  });
  __builtin_amdgcn_s_waitcnt(xd_wait_vm(0));

  const uint32_t nt0 = bn + wn * WN, mt0 = bm + wm * WM;
  const uint32_t q = lane >> 4, c = lane & 15;
  if constexpr (EPI == kEpiQkvRope) {
    __syncthreads();  // every wave is done reading the weight ring, which the staging reuses
    if (mt0 * 16 >= m) return;  // this wave's rows are all padding
    // D layout: lane l, element e holds column 16 i + 4 (l / 16) + e of the
    // head and row 16 j + l % 16 of the wave's 64 rows.
    uint32_t* rows_lds = reinterpret_cast<uint32_t*>(lds_raw) + (uint32_t)wave * 64 * kQkPitch;
#pragma unroll
    for (int j = 0; j < WM; ++j)
#pragma unroll
      for (int i = 0; i < WN; ++i) {
        const uint2 v = make_uint2(f32_to_bf16(acc[i][j][0]) | (f32_to_bf16(acc[i][j][1]) << 16),
                                   f32_to_bf16(acc[i][j][2]) | (f32_to_bf16(acc[i][j][3]) << 16));
        *reinterpret_cast<uint2*>(rows_lds + (16 * j + c) * kQkPitch + 8 * i + 2 * q) = v;
      }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t row = mt0 * 16 + lane;
    if (row < m)
      qknorm_rope_kv_head<32, true>(reinterpret_cast<const qk_u32x4*>(rows_lds + lane * kQkPitch), row,
                              gx * 2 + wn, qa, row_slot);
    return;
  }
  if (mt0 * 16 >= m) return;  // this wave's rows are all padding
  if constexpr (EPI == FH_EPI_SWIGLU) {
    bool bad = false;
#pragma unroll
    for (int p = 0; p < WN / 2; ++p) {
      const uint32_t col = ((nt0 + 2 * p) / 2) * 16 + 4 * q;
#pragma unroll
      for (int j = 0; j < WM; ++j) {
        const uint32_t row = (mt0 + j) * 16 + c;
        if (row >= m) continue;
        uint32_t y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          y[e] = swiglu_bf16(round_bf16(acc[2 * p][j][e]), round_bf16(acc[2 * p + 1][j][e]), bad);
        uint2 v = make_uint2(y[0] | (y[1] << 16), y[2] | (y[3] << 16));
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + act_offset_m(row, col, out_mtiles)) = v;
      }
    }
    if (bad) raise_error(err, ERR_NONFINITE);
  } else {
#pragma unroll
    for (int i = 0; i < WN; ++i) {
      const uint32_t n = (nt0 + i) * 16 + 4 * q;
#pragma unroll
      for (int j = 0; j < WM; ++j) {
        const uint32_t row = (mt0 + j) * 16 + c;
        if (row >= m) continue;
        const uint64_t o = (uint64_t)row * ldo + n;
        if constexpr (EPI == FH_EPI_F32) {
          *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(out) + o) = acc[i][j];
        } else if constexpr (EPI == FH_EPI_BF16) {
          uint2 v = make_uint2(f32_to_bf16(acc[i][j][0]) | (f32_to_bf16(acc[i][j][1]) << 16),
                               f32_to_bf16(acc[i][j][2]) | (f32_to_bf16(acc[i][j][3]) << 16));
          *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + o) = v;
        } else {
          const uint2 rv = *reinterpret_cast<const uint2*>(residual + o);
          const float r0 = lo_bf16(rv.x), r1 = hi_bf16(rv.x), r2 = lo_bf16(rv.y), r3 = hi_bf16(rv.y);
          uint2 v = make_uint2(f32_to_bf16((0.0f + acc[i][j][0]) + r0) | (f32_to_bf16((0.0f + acc[i][j][1]) + r1) << 16),
                               f32_to_bf16((0.0f + acc[i][j][2]) + r2) | (f32_to_bf16((0.0f + acc[i][j][3]) + r3) << 16));
          *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + o) = v;
        }
      }
    }
  }
}

}  // namespace

hipError_t launch_gemm_qkv_rope(const uint16_t* x_tiled, const uint16_t* w_tiled, uint32_t m, uint32_t n, uint32_t k,
                                const QkvRopeArgs& qa, hipStream_t s) {
  const uint32_t mtiles = act_mtiles(m);
  if (m <= kStreamedRows || n % (16 * kBigTiles) != 0 || k % 32 != 0 || mtiles % kBigTiles != 0 ||
      n != (qa.qh + 2 * qa.kvh) * 128)
    return hipErrorInvalidValue;
  const dim3 grid(n / (16 * kBigTiles), mtiles / kBigTiles);
  hipLaunchKernelGGL((gemm_large_xd_kernel<kEpiQkvRope>), grid, dim3(512), 0, s, x_tiled, w_tiled, m, mtiles, k / 32,
                     (const uint16_t*)nullptr, (void*)nullptr, 0u, 0u, qa, (uint32_t*)nullptr);
  return hipGetLastError();
}

hipError_t launch_gemm_large(const uint16_t* x_tiled, const uint16_t* w_tiled, uint32_t m, uint32_t n, uint32_t k,
                             uint32_t epilogue, const uint16_t* residual, void* out, uint32_t ldo, uint32_t* err,
                             hipStream_t s) {
  // Up to kStreamedRows rows the weight-streaming kernel is faster: it runs
  // 32-row chunks of the batch against the same weight tiles (a prefill
  // chunk of 17..32 rows when row_capacity < 32, a speculative verify batch).
  if (m <= kStreamedRows) return launch_gemm(x_tiled, w_tiled, m, n, k, epilogue, 1, residual, out, ldo, err, s);
  if (n % (16 * kBlockTiles) != 0 || k % 32 != 0) return hipErrorInvalidValue;
  const uint32_t mtiles = act_mtiles(m);
  const uint32_t out_mtiles = epilogue == FH_EPI_SWIGLU ? act_mtiles(m) : 0u;
  const uint32_t kb = k / 32;
  if (n % (16 * kBigTiles) == 0 && mtiles % kBigTiles == 0) {
    const dim3 grid(n / (16 * kBigTiles), mtiles / kBigTiles);
#define FH_BIG(E)                                                                                           \
  hipLaunchKernelGGL((gemm_large_xd_kernel<E>), grid, dim3(512), 0, s, x_tiled, w_tiled, m, mtiles, kb, residual, \
                     out, ldo, out_mtiles, QkvRopeArgs{}, err)
    switch (epilogue) {
      case FH_EPI_BF16: FH_BIG(FH_EPI_BF16); break;
      case FH_EPI_RESIDUAL: FH_BIG(FH_EPI_RESIDUAL); break;
      case FH_EPI_SWIGLU: FH_BIG(FH_EPI_SWIGLU); break;
      case FH_EPI_F32: FH_BIG(FH_EPI_F32); break;
      default: return hipErrorInvalidValue;
    }
#undef FH_BIG
    return hipGetLastError();
  }
  const dim3 grid(n / (16 * kBlockTiles), mtiles / kBlockTiles);
  switch (epilogue) {
    case FH_EPI_BF16:
      hipLaunchKernelGGL(gemm_large_kernel<FH_EPI_BF16>, grid, dim3(256), 0, s, x_tiled, w_tiled, m, mtiles, kb,
                         residual, out, ldo, out_mtiles, err);
      break;
    case FH_EPI_RESIDUAL:
      hipLaunchKernelGGL(gemm_large_kernel<FH_EPI_RESIDUAL>, grid, dim3(256), 0, s, x_tiled, w_tiled, m, mtiles, kb,
                         residual, out, ldo, out_mtiles, err);
      break;
    case FH_EPI_SWIGLU:
      hipLaunchKernelGGL(gemm_large_kernel<FH_EPI_SWIGLU>, grid, dim3(256), 0, s, x_tiled, w_tiled, m, mtiles, kb,
                         residual, out, ldo, out_mtiles, err);
      break;
    case FH_EPI_F32:
      hipLaunchKernelGGL(gemm_large_kernel<FH_EPI_F32>, grid, dim3(256), 0, s, x_tiled, w_tiled, m, mtiles, kb,
                         residual, out, ldo, out_mtiles, err);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace fh
