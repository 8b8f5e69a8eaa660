// K4 paged GQA decode attention for gfx950: split-context partitions with an
// ordered merge.
//
// Reference semantics (device/qwen3-all-kernels-v1/src/paged_decode.rs:222-572):
// for a query row at position p, keys t = 0..p through the row's page table,
// score = (q . k_t) * f32(0x3db504f3), softmax, out = bf16(n / l). The
// reference's split variant (device/qwen3-tp-c1-split8-attention-kernels-v21,
// README.md:42-80) partitions the context, keeps an FP32 state (m, l, n[128])
// per partition, merges the partitions in ascending order, then divides and
// narrows once. This kernel pair keeps that contract with 32-page (512-token)
// partitions and GQA sharing: one workgroup serves the G query heads of one KV
// head, so every K/V page is read from HBM once per token row.
//
// Partition kernel, grid (partition, kv_head, row), 4 waves; wave w walks 8
// consecutive pages of the partition, one page (16 tokens) per iteration,
// with the next page's K and V loads in flight while the current page is
// computed:
//   QK^T on MFMA: S^T = K Q^T, the 16-token K page as the A operand straight
//   from the paged cache (lane l holds token l % 16; MFMA i covers dims
//   32 i .. 32 i + 31, so each load instruction reads 64 contiguous bytes of
//   every token), the G queries as the B operand (registers).
//   Online softmax per page (page max, rescale, exp, page sum).
//   PV on VALU: lane l owns output dims 2l, 2l+1; a token's V row is one
//   coalesced 256-byte wave load.
// The four wave states are merged in wave order. A row whose context fits
// one partition is finished here (divide, narrow, store); longer rows leave
// partition states for the merge kernel.
// Merge kernel: one wave per (row, query head). Partition weights
// w_p = exp(m_p - M) with M the maximum over partitions, then l and n are
// summed over partitions in ascending order, divided, narrowed once.
#include "common.hpp"
#include "kernels.hpp"

namespace fh {

namespace {

constexpr int kAttnThreads = 256;
constexpr uint32_t kWavePages = kAttnSplitPages / 4;
constexpr uint32_t kScaleBits = 0x3db504f3u;  // f32 1/sqrt(128), paged_decode.rs:31-35

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Stores one finished head output (dims 2*lane, 2*lane+1) in either layout.
__device__ __forceinline__ void store_head(uint16_t* out, bool tiled, uint32_t r, uint32_t qh, uint32_t head, int lane,
                                          uint32_t o0, uint32_t o1) {
  const uint32_t col = head * 128 + 2 * lane;
  const uint32_t word = o0 | (o1 << 16);
  if (tiled)
    *reinterpret_cast<uint32_t*>(out + act_offset(r, col)) = word;
  else
    reinterpret_cast<uint32_t*>(out + ((uint64_t)r * qh + head) * 128)[lane] = word;
}

template <int G>
__global__ __launch_bounds__(kAttnThreads) void attn_partition_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    const uint32_t* __restrict__ positions, const uint32_t* __restrict__ table, float* __restrict__ part,
    uint16_t* __restrict__ out, uint32_t out_tiled, uint32_t qh, uint32_t kvh, uint32_t stride, uint32_t pages,
    uint32_t context, uint32_t smax, uint32_t* err) {
  const uint32_t split = blockIdx.x, h = blockIdx.y, r = blockIdx.z;
  const uint32_t pos = positions[r];
  if (pos >= context || pos / 16 >= stride) {
    if (split == 0 && h == 0 && threadIdx.x == 0) raise_error(err, ERR_POSITION);
    return;
  }
  const uint32_t ctx = pos + 1;
  const uint32_t row_pages = (ctx + 15) / 16;
  const uint32_t p0 = split * kAttnSplitPages;
  if (p0 >= row_pages) return;  // uniform per workgroup
  const uint32_t nsplit = (row_pages + kAttnSplitPages - 1) / kAttnSplitPages;

  __shared__ float pbuf[4][16][G];
  __shared__ float wstat[4][2][G];
  __shared__ float wacc[4][G][128];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g16 = lane >> 4, r16 = lane & 15;
  const float scale = __builtin_bit_cast(float, kScaleBits);
  const float kNegInf = -__builtin_inff();
  const uint32_t* trow = table + (uint64_t)r * stride;

  // B operand: query head h*G + r16 (zero for r16 >= G); MFMA i, lane group
  // g16 covers dims 32*i + 8*g16 .. +7.
  u32x4 qv[4];
  if (r16 < G) {
    const uint16_t* qp = q + ((uint64_t)r * qh + h * G + r16) * 128 + 8 * g16;
#pragma unroll
    for (int i = 0; i < 4; ++i) qv[i] = *reinterpret_cast<const u32x4*>(qp + 32 * i);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) qv[i] = u32x4{0u, 0u, 0u, 0u};
  }

  const uint32_t wp0 = p0 + wave * kWavePages;
  const uint32_t wp1 = min(min(wp0 + kWavePages, p0 + kAttnSplitPages), row_pages);
  const int np = wp1 > wp0 ? (int)(wp1 - wp0) : 0;
  const uint32_t vstride = kvh * 64;  // dwords between consecutive slots of one head

  float m[G], l[G], acc[G][2];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNegInf;
    l[g] = 0.f;
    acc[g][0] = acc[g][1] = 0.f;
  }
  bool bad = false;

  u32x4 kcur[4], knext[4];
  uint32_t vcur[16], vnext[16];
  auto load_page = [&](uint32_t page, u32x4* kd, uint32_t* vd) {
    uint32_t phys = trow[page];
    if (phys >= pages) {
      bad = true;
      phys = 0;
    }
    const uint16_t* kp = kc + (((uint64_t)phys * 16 + r16) * kvh + h) * 128 + 8 * g16;
#pragma unroll
    for (int i = 0; i < 4; ++i) kd[i] = *reinterpret_cast<const u32x4*>(kp + 32 * i);
    const uint32_t* vp = reinterpret_cast<const uint32_t*>(vc + (((uint64_t)phys * 16) * kvh + h) * 128) + lane;
#pragma unroll
    for (int e = 0; e < 16; ++e) vd[e] = vp[e * vstride];
  };

  if (np > 0) load_page(wp0, kcur, vcur);
  for (int j = 0; j < np; ++j) {
    const uint32_t page = wp0 + j;
    if (j + 1 < np) load_page(page + 1, knext, vnext);

    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kcur[i]),
                                                 __builtin_bit_cast(bf16x8, qv[i]), s, 0, 0, 0);
    // Lane holds query r16 for tokens 4*g16 + e of this page.
    const uint32_t t0 = page * 16;
    float sc[4];
    float pm = kNegInf;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool valid = t0 + 4 * g16 + e < ctx;
      sc[e] = valid ? s[e] * scale : kNegInf;
      bad |= valid && !is_finite_f32(sc[e]);
      pm = fmaxf(pm, sc[e]);
    }
    pm = fmaxf(pm, __shfl_xor(pm, 16, 64));
    pm = fmaxf(pm, __shfl_xor(pm, 32, 64));
    // New running max per head (wave-uniform) and the rescale factors.
    float mnew[G], alpha[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      mnew[g] = fmaxf(m[g], lane_bcast(pm, g));
      alpha[g] = expf(m[g] - mnew[g]);  // m = -inf on the first page: alpha = 0
    }
    float mine = mnew[0];
#pragma unroll
    for (int g = 1; g < G; ++g) mine = r16 == g ? mnew[g] : mine;
    float ps = 0.f;
    float pr[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      pr[e] = sc[e] > kNegInf ? expf(sc[e] - mine) : 0.f;
      ps += pr[e];
    }
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    if (r16 < G) {
#pragma unroll
      for (int e = 0; e < 4; ++e) pbuf[wave][4 * g16 + e][r16] = pr[e];
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      l[g] = l[g] * alpha[g] + lane_bcast(ps, g);
      acc[g][0] *= alpha[g];
      acc[g][1] *= alpha[g];
      m[g] = mnew[g];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t valid_tokens = min(16u, ctx - t0);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const uint32_t v = (uint32_t)e < valid_tokens ? vcur[e] : 0u;
      const float v0 = lo_bf16(v), v1 = hi_bf16(v);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float p = pbuf[wave][e][g];
        acc[g][0] = fmaf(p, v0, acc[g][0]);
        acc[g][1] = fmaf(p, v1, acc[g][1]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int i = 0; i < 4; ++i) kcur[i] = knext[i];
#pragma unroll
    for (int e = 0; e < 16; ++e) vcur[e] = vnext[e];
  }

  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      wstat[wave][0][g] = m[g];
      wstat[wave][1][g] = l[g];
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    wacc[wave][g][2 * lane] = acc[g][0];
    wacc[wave][g][2 * lane + 1] = acc[g][1];
  }
  __syncthreads();

  if (nsplit == 1) {
    // Whole context in this partition: merge the waves, divide, narrow, store.
    for (int g = wave; g < G; g += 4) {
      float M = wstat[0][0][g];
#pragma unroll
      for (int w = 1; w < 4; ++w) M = fmaxf(M, wstat[w][0][g]);
      float L = 0.f, n0 = 0.f, n1 = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float lw = wstat[w][1][g];
        if (lw > 0.f) {
          const float f = expf(wstat[w][0][g] - M);
          L += lw * f;
          n0 += wacc[w][g][2 * lane] * f;
          n1 += wacc[w][g][2 * lane + 1] * f;
        }
      }
      const uint32_t o0 = f32_to_bf16(n0 / L), o1 = f32_to_bf16(n1 / L);
      bad |= !(L > 0.f) | ((o0 & 0x7f80u) == 0x7f80u) | ((o1 & 0x7f80u) == 0x7f80u);
      store_head(out, out_tiled != 0, r, qh, h * G + g, lane, o0, o1);
    }
  } else {
    for (int idx = threadIdx.x; idx < G * (int)kAttnPartialFloats; idx += kAttnThreads) {
      const int g = idx / (int)kAttnPartialFloats, c = idx % (int)kAttnPartialFloats;
      float M = wstat[0][0][g];
#pragma unroll
      for (int w = 1; w < 4; ++w) M = fmaxf(M, wstat[w][0][g]);
      float v;
      if (c == 0) {
        v = M;
      } else {
        v = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float lw = wstat[w][1][g];
          if (lw > 0.f) v += (c == 1 ? lw : wacc[w][g][c - 2]) * expf(wstat[w][0][g] - M);
        }
      }
      part[(((uint64_t)r * qh + h * G + g) * smax + split) * kAttnPartialFloats + c] = v;
    }
  }
  if (bad) raise_error(err, ERR_NONFINITE);
}

__global__ __launch_bounds__(kAttnThreads) void attn_merge_kernel(const float* __restrict__ part,
                                                                  const uint32_t* __restrict__ positions,
                                                                  uint16_t* __restrict__ out, uint32_t out_tiled,
                                                                  uint32_t rows, uint32_t qh, uint32_t context,
                                                                  uint32_t smax, uint32_t* err) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t id = blockIdx.x * 4 + wave;
  const uint32_t r = id / qh, head = id % qh;
  if (r >= rows) return;
  const uint32_t pos = positions[r];
  if (pos >= context) return;  // reported by the partition kernel
  const uint32_t row_pages = (pos + 16) / 16;
  const uint32_t ns = (row_pages + kAttnSplitPages - 1) / kAttnSplitPages;
  if (ns == 1) return;  // finished by the partition kernel
  const float* p = part + ((uint64_t)r * qh + head) * smax * kAttnPartialFloats;
  // Lane s < ns holds partition s's (m, l).
  const float ms = lane < (int)ns ? p[(uint64_t)lane * kAttnPartialFloats] : -__builtin_inff();
  const float M = wave_max(ms);
  const float ws = lane < (int)ns ? expf(ms - M) : 0.f;
  const float lw = lane < (int)ns ? p[(uint64_t)lane * kAttnPartialFloats + 1] * ws : 0.f;
  float L = 0.f, n0 = 0.f, n1 = 0.f;
  for (uint32_t s0 = 0; s0 < ns; s0 += 8) {
    // Eight partitions' numerators in flight, then added in ascending order.
    float a0[8], a1[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const uint32_t sp = s0 + u;
      const float* ps = p + (uint64_t)sp * kAttnPartialFloats;
      a0[u] = sp < ns ? ps[2 + 2 * lane] : 0.f;
      a1[u] = sp < ns ? ps[3 + 2 * lane] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const uint32_t sp = s0 + u;
      if (sp < ns) {
        const float w = lane_bcast(ws, (int)sp);
        L += lane_bcast(lw, (int)sp);
        n0 += a0[u] * w;
        n1 += a1[u] * w;
      }
    }
  }
  const uint32_t o0 = f32_to_bf16(n0 / L), o1 = f32_to_bf16(n1 / L);
  store_head(out, out_tiled != 0, r, qh, head, lane, o0, o1);
  if (!(L > 0.f) || ((o0 & 0x7f80u) == 0x7f80u) || ((o1 & 0x7f80u) == 0x7f80u)) raise_error(err, ERR_NONFINITE);
}

template <int G>
void launch_partition(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, const uint32_t* positions,
                      const uint32_t* table, float* part, uint16_t* out, uint32_t out_tiled, uint32_t rows,
                      uint32_t qh, uint32_t kvh, uint32_t stride, uint32_t pages, uint32_t context, uint32_t smax,
                      uint32_t* err, hipStream_t s) {
  hipLaunchKernelGGL((attn_partition_kernel<G>), dim3(smax, kvh, rows), dim3(kAttnThreads), 0, s, q, kc, vc,
                     positions, table, part, out, out_tiled, qh, kvh, stride, pages, context, smax, err);
}

}  // namespace

hipError_t launch_attention_partial(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                    const uint32_t* positions, const uint32_t* table, float* partials, uint16_t* out,
                                    uint32_t out_tiled, uint32_t rows, uint32_t qh, uint32_t kvh, uint32_t stride,
                                    uint32_t pages, uint32_t context, uint32_t* err, hipStream_t s) {
  const uint32_t smax = attn_max_splits(context);
  switch (qh / kvh) {
    case 1: launch_partition<1>(q, k_cache, v_cache, positions, table, partials, out, out_tiled, rows, qh, kvh, stride, pages, context, smax, err, s); break;
    case 2: launch_partition<2>(q, k_cache, v_cache, positions, table, partials, out, out_tiled, rows, qh, kvh, stride, pages, context, smax, err, s); break;
    case 4: launch_partition<4>(q, k_cache, v_cache, positions, table, partials, out, out_tiled, rows, qh, kvh, stride, pages, context, smax, err, s); break;
    case 8: launch_partition<8>(q, k_cache, v_cache, positions, table, partials, out, out_tiled, rows, qh, kvh, stride, pages, context, smax, err, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_attention_merge(const float* partials, const uint32_t* positions, uint16_t* out,
                                  uint32_t out_tiled, uint32_t rows, uint32_t qh, uint32_t context, uint32_t* err,
                                  hipStream_t s) {
  const uint32_t smax = attn_max_splits(context);
  const uint32_t waves = rows * qh;
  hipLaunchKernelGGL(attn_merge_kernel, dim3((waves + 3) / 4), dim3(kAttnThreads), 0, s, partials, positions, out,
                     out_tiled, rows, qh, context, smax, err);
  return hipGetLastError();
}

}  // namespace fh
