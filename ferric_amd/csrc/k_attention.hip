// K4 paged GQA decode attention for gfx950: split-context partials with an
// ordered merge.
//
// Reference semantics (device/qwen3-all-kernels-v1/src/paged_decode.rs:222-572):
// for every query row at position p, keys t = 0..p through the row's page
// table, score = (q . k_t) * f32(0x3db504f3), online softmax, out = bf16(n / l).
// The reference's split variant (device/qwen3-tp-c1-split8-attention-kernels-v21,
// README.md:42-80) partitions the context, keeps (m, l, n[128]) per
// partition, and merges partitions in ascending order before one division and
// one narrowing. This kernel pair follows that contract with 256-token
// partitions (16 pages) and GQA sharing: one workgroup serves all G query
// heads of one KV head, so each K/V page is read from HBM once per row.
//
// Partial kernel, grid (split, kv_head, row), 4 waves x 64 tokens:
//   QK^T on MFMA: S^T = K Q^T with the K page as the A operand loaded straight
//   from the paged cache (lane l reads 64 contiguous bytes of token l % 16) and
//   the G queries as the B operand (registers).
//   Softmax per wave (max, exp, sum over its 64 tokens), probabilities to LDS.
//   PV on VALU: lane l owns output dims 2l, 2l+1; each token's V row is one
//   coalesced 256-byte wave load.
//   The four wave states are merged in wave order into the partition state.
// Merge kernel: one wave per (row, query head), partitions in ascending order.
#include "common.hpp"
#include "kernels.hpp"

namespace fh {

namespace {

constexpr int kAttnThreads = 256;
constexpr uint32_t kScaleBits = 0x3db504f3u;  // f32 1/sqrt(128), paged_decode.rs:31-35

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int G>
__global__ __launch_bounds__(kAttnThreads) void attn_partial_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    const uint32_t* __restrict__ positions, const uint32_t* __restrict__ table, float* __restrict__ part,
    uint32_t qh, uint32_t kvh, uint32_t stride, uint32_t pages, uint32_t context, uint32_t smax, uint32_t* err) {
  const uint32_t split = blockIdx.x, h = blockIdx.y, r = blockIdx.z;
  const uint32_t pos = positions[r];
  if (pos >= context || pos / 16 >= stride) {
    if (split == 0 && h == 0 && threadIdx.x == 0) raise_error(err, ERR_POSITION);
    return;
  }
  const uint32_t ctx = pos + 1;
  const uint32_t start = split * kAttnSplitTokens;
  if (start >= ctx) return;  // uniform per workgroup

  __shared__ float pbuf[4][64][G];
  __shared__ float wstat[4][2][G];
  __shared__ float wacc[4][G][128];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g16 = lane >> 4, r16 = lane & 15;
  const float scale = __builtin_bit_cast(float, kScaleBits);
  const uint32_t* trow = table + (uint64_t)r * stride;
  const float kNegInf = -__builtin_inff();

  // B operand: query head h*G + r16 (zero for r16 >= G), dims 32*g16 + 8*i + e.
  u32x4 qv[4];
  if (r16 < G) {
    const u32x4* qp = reinterpret_cast<const u32x4*>(q + ((uint64_t)r * qh + h * G + r16) * 128 + 32 * g16);
#pragma unroll
    for (int i = 0; i < 4; ++i) qv[i] = qp[i];
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) qv[i] = u32x4{0u, 0u, 0u, 0u};
  }

  const uint32_t wstart = start + wave * 64;
  bool page_bad = false;
  u32x4 kv[4][4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t page_start = wstart + 16 * p;
    if (page_start < ctx) {
      uint32_t phys = trow[page_start >> 4];
      if (phys >= pages) {
        page_bad = true;
        phys = 0;
      }
      const u32x4* kp =
          reinterpret_cast<const u32x4*>(kc + (((uint64_t)phys * 16 + r16) * kvh + h) * 128 + 32 * g16);
#pragma unroll
      for (int i = 0; i < 4; ++i) kv[p][i] = __builtin_nontemporal_load(kp + i);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) kv[p][i] = u32x4{0u, 0u, 0u, 0u};
    }
  }
  if (page_bad) raise_error(err, ERR_PAGE);

  // Scores: lane holds query r16, tokens wstart + 16p + 4*g16 + e.
  float sv[4][4];
  float mx = kNegInf;
  bool bad = false;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kv[p][i]),
                                                   __builtin_bit_cast(bf16x8, qv[i]), acc, 0, 0, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t t = wstart + 16 * p + 4 * g16 + e;
      float sc = kNegInf;
      if (t < ctx) {
        sc = acc[e] * scale;
        bad |= !is_finite_f32(sc);
      }
      sv[p][e] = sc;
      mx = fmaxf(mx, sc);
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  float l = 0.f;
#pragma unroll
  for (int p = 0; p < 4; ++p)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float sc = sv[p][e];
      float pr = sc > kNegInf ? expf(sc - mx) : 0.f;
      l += pr;
      if (r16 < G) pbuf[wave][16 * p + 4 * g16 + e][r16] = pr;
    }
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (lane < G) {
    wstat[wave][0][lane] = mx;
    wstat[wave][1][lane] = l;
  }
  __syncthreads();

  // PV: lane owns dims 2*lane, 2*lane + 1.
  float acc[G][2];
#pragma unroll
  for (int g = 0; g < G; ++g) acc[g][0] = acc[g][1] = 0.f;
  const uint32_t n_valid = ctx > wstart ? min(64u, ctx - wstart) : 0u;
  for (uint32_t p = 0; p < 4; ++p) {
    const uint32_t base_t = p * 16;
    if (base_t >= n_valid) break;
    uint32_t phys = trow[(wstart + base_t) >> 4];
    if (phys >= pages) phys = 0;
    const uint32_t* vp = reinterpret_cast<const uint32_t*>(vc + (((uint64_t)phys * 16) * kvh + h) * 128) + lane;
    const uint32_t tok_stride = kvh * 64;  // dwords between consecutive slots of one head
    const uint32_t cnt = min(16u, n_valid - base_t);
    uint32_t vv[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) vv[e] = (uint32_t)e < cnt ? __builtin_nontemporal_load(vp + e * tok_stride) : 0u;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      if ((uint32_t)e < cnt) {
        const float v0 = lo_bf16(vv[e]), v1 = hi_bf16(vv[e]);
        const float* pp = &pbuf[wave][base_t + e][0];
#pragma unroll
        for (int g = 0; g < G; ++g) {
          acc[g][0] = fmaf(pp[g], v0, acc[g][0]);
          acc[g][1] = fmaf(pp[g], v1, acc[g][1]);
        }
      }
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    wacc[wave][g][2 * lane] = acc[g][0];
    wacc[wave][g][2 * lane + 1] = acc[g][1];
  }
  __syncthreads();

  // Partition state = ordered merge of the four wave states.
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
        if (lw > 0.f) {
          const float f = expf(wstat[w][0][g] - M);
          v += (c == 1 ? lw : wacc[w][g][c - 2]) * f;
        }
      }
    }
    part[(((uint64_t)r * qh + h * G + g) * smax + split) * kAttnPartialFloats + c] = v;
  }
  if (bad) raise_error(err, ERR_NONFINITE);
}

// Ordered merge (v21 README.md:71-80): seed with partition 0, then for
// p = 1..: m' = max(m, m_p); l = l e^(m-m') + l_p e^(m_p-m'); n likewise.
__global__ __launch_bounds__(kAttnThreads) void attn_merge_kernel(const float* __restrict__ part,
                                                                  const uint32_t* __restrict__ positions,
                                                                  uint16_t* __restrict__ out, uint32_t rows,
                                                                  uint32_t qh, uint32_t context, uint32_t smax,
                                                                  uint32_t* err) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t id = blockIdx.x * 4 + wave;
  const uint32_t r = id / qh, head = id % qh;
  if (r >= rows) return;
  const uint32_t pos = positions[r];
  if (pos >= context) return;  // reported by the partial kernel
  const uint32_t ns = (pos + kAttnSplitTokens) / kAttnSplitTokens;
  const float* p = part + ((uint64_t)r * qh + head) * smax * kAttnPartialFloats;
  float m = p[0], l = p[1];
  float n0 = p[2 + 2 * lane], n1 = p[3 + 2 * lane];
  for (uint32_t sp = 1; sp < ns; ++sp) {
    const float* ps = p + (uint64_t)sp * kAttnPartialFloats;
    const float ms = ps[0], ls = ps[1];
    const float nm = fmaxf(m, ms);
    const float pw = expf(m - nm), cw = expf(ms - nm);
    l = l * pw + ls * cw;
    n0 = n0 * pw + ps[2 + 2 * lane] * cw;
    n1 = n1 * pw + ps[3 + 2 * lane] * cw;
    m = nm;
  }
  const uint32_t o0 = f32_to_bf16(n0 / l), o1 = f32_to_bf16(n1 / l);
  reinterpret_cast<uint32_t*>(out + ((uint64_t)r * qh + head) * 128)[lane] = o0 | (o1 << 16);
  if (!(l > 0.f) || ((o0 & 0x7f80u) == 0x7f80u) || ((o1 & 0x7f80u) == 0x7f80u)) raise_error(err, ERR_NONFINITE);
}

template <int G>
void launch_partial(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, const uint32_t* positions,
                    const uint32_t* table, float* part, uint32_t rows, uint32_t qh, uint32_t kvh, uint32_t stride,
                    uint32_t pages, uint32_t context, uint32_t smax, uint32_t* err, hipStream_t s) {
  hipLaunchKernelGGL((attn_partial_kernel<G>), dim3(smax, kvh, rows), dim3(kAttnThreads), 0, s, q, kc, vc, positions,
                     table, part, qh, kvh, stride, pages, context, smax, err);
}

}  // namespace

hipError_t launch_attention_partial(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                    const uint32_t* positions, const uint32_t* table, float* partials, uint32_t rows,
                                    uint32_t qh, uint32_t kvh, uint32_t stride, uint32_t pages, uint32_t context,
                                    uint32_t* err, hipStream_t s) {
  const uint32_t smax = attn_max_splits(context);
  switch (qh / kvh) {
    case 1: launch_partial<1>(q, k_cache, v_cache, positions, table, partials, rows, qh, kvh, stride, pages, context, smax, err, s); break;
    case 2: launch_partial<2>(q, k_cache, v_cache, positions, table, partials, rows, qh, kvh, stride, pages, context, smax, err, s); break;
    case 4: launch_partial<4>(q, k_cache, v_cache, positions, table, partials, rows, qh, kvh, stride, pages, context, smax, err, s); break;
    case 8: launch_partial<8>(q, k_cache, v_cache, positions, table, partials, rows, qh, kvh, stride, pages, context, smax, err, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_attention_merge(const float* partials, const uint32_t* positions, uint16_t* out, uint32_t rows,
                                  uint32_t qh, uint32_t context, uint32_t* err, hipStream_t s) {
  const uint32_t smax = attn_max_splits(context);
  const uint32_t waves = rows * qh;
  hipLaunchKernelGGL(attn_merge_kernel, dim3((waves + 3) / 4), dim3(kAttnThreads), 0, s, partials, positions, out, rows,
                     qh, context, smax, err);
  return hipGetLastError();
}

}  // namespace fh
