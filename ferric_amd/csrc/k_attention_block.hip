// K4 for prefill chunks: causal attention of blocks of consecutive rows of
// one sequence.
//
// Reference semantics: the batched prefill runs the paged decode attention
// per row with that row's position (device/qwen3-all-kernels-v1/src/
// paged_decode.rs:222-572, and prefill.rs:153 for one contiguous sequence):
// keys t = 0..p of the row's sequence, score = (q . k_t) * f32(0x3db504f3),
// softmax, out = bf16(n / l). A prefill chunk holds runs of rows of the same
// sequence at consecutive positions whose page lists extend one another; the
// host groups such a run into blocks of up to 64 / G rows and this kernel
// reads each K/V page once per block instead of once per row.
//
// Grid (block, KV head), 4 waves. A wave owns 16 query vectors: 16 / G rows
// times the G query heads of the KV head (vector j: row j / G, head j % G).
// Per 16-token page, shared by the workgroup through LDS (double-buffered,
// the next page's loads in flight while this one is used):
//   S^T = K Q^T on v_mfma_f32_16x16x32_bf16 (K page re-laid through a padded
//   LDS tile into the A operand, the queries as the B operand), scaled and
//   masked by each row's position (t <= p);
//   online softmax per query vector: m' = max(m, page max),
//   alpha = exp(m - m'), l = l alpha + sum exp(s - m'), n = n alpha + P V
//   (the recurrence of the reference taken one page at a time, FP32);
//   PV on VALU in FP32: lane l owns dims 2l, 2l+1 of the 16 vectors.
// Finally out = bf16(n / l) for each valid row.
#include "common.hpp"
#include "kernels.hpp"

namespace fh {

namespace {

constexpr uint32_t kScaleBitsB = 0x3db504f3u;  // f32 1/sqrt(128), paged_decode.rs:31-35

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float exp2_based(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int G>
__global__ __launch_bounds__(256) void attn_block_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    const uint32_t* __restrict__ positions, const uint32_t* __restrict__ table, const uint32_t* __restrict__ blocks,
    uint16_t* __restrict__ out, uint32_t out_mtiles, uint32_t qh, uint32_t kvh, uint32_t stride, uint32_t pages,
    uint32_t context, uint32_t* err) {
  constexpr int kRowsPerWave = 16 / G;
  static_assert(16 % G == 0, "16 query vectors per wave");
  const uint32_t desc = blocks[blockIdx.x];
  const uint32_t row0 = desc & 0xffffu, nrows = desc >> 16;
  const uint32_t h = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t last = row0 + nrows - 1;
  const uint32_t pmax = positions[last];  // rows of a block have consecutive positions
  if (pmax >= context || pmax / 16 >= stride) {
    if (h == 0 && threadIdx.x == 0) raise_error(err, ERR_POSITION);
    return;
  }
  const uint32_t npages = pmax / 16 + 1;
  const uint32_t* trow = table + (uint64_t)last * stride;

  __shared__ u32x4 ktile[2][16][17];
  __shared__ u32x4 vtile[2][16][16];
  __shared__ float pbuf[4][16][16];  // [wave][key][query vector]

  const int j = lane & 15, g16 = lane >> 4;
  const uint32_t rj = wave * kRowsPerWave + j / G;
  const bool qvalid = rj < nrows;
  const uint32_t qpos = qvalid ? positions[row0 + rj] : 0u;
  u32x4 qv[4];
  if (qvalid) {
    const uint16_t* qp = q + ((uint64_t)(row0 + rj) * qh + h * G + j % G) * 128 + 8 * g16;
#pragma unroll
    for (int i = 0; i < 4; ++i) qv[i] = *reinterpret_cast<const u32x4*>(qp + 32 * i);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) qv[i] = u32x4{0u, 0u, 0u, 0u};
  }

  bool bad = false;
  auto phys = [&](uint32_t pi) {
    uint32_t ph = pi < npages ? trow[pi] : 0u;
    if (ph >= pages) {
      bad = true;
      ph = 0;
    }
    return ph;
  };
  // Loader mapping: thread t copies 16 bytes (dims 8 c .. 8 c + 7) of token
  // t / 16 of the page, for K and for V.
  const uint32_t lt = threadIdx.x >> 4, lc = threadIdx.x & 15;
  auto src = [&](uint32_t ph) { return (((uint64_t)ph * 16 + lt) * kvh + h) * 128 + 8 * lc; };
  uint32_t ph_next = phys(1), ph_next2 = phys(2);
  u32x4 kreg, vreg;
  {
    const uint64_t o = src(phys(0));
    kreg = *reinterpret_cast<const u32x4*>(kc + o);
    vreg = *reinterpret_cast<const u32x4*>(vc + o);
  }

  const float scale = __builtin_bit_cast(float, kScaleBitsB);
  const float kNegInf = -__builtin_inff();
  float m_run = kNegInf, l_run = 0.f;
  float acc[16][2];
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v][0] = acc[v][1] = 0.f;

  for (uint32_t p = 0; p < npages; ++p) {
    const int b = p & 1;
    ktile[b][lt][lc] = kreg;
    vtile[b][lt][lc] = vreg;
    if (p + 1 < npages) {
      const uint64_t o = src(ph_next);
      kreg = *reinterpret_cast<const u32x4*>(kc + o);
      vreg = *reinterpret_cast<const u32x4*>(vc + o);
    }
    ph_next = ph_next2;
    ph_next2 = phys(p + 3);
    __syncthreads();

    // Scores: lane l, element e holds key 4 g16 + e of the page for vector j.
    u32x4 ka[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ka[i] = ktile[b][j][4 * i + g16];
    f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ka[i]),
                                                    __builtin_bit_cast(bf16x8, qv[i]), sacc, 0, 0, 0);
    float sv[4];
    float pm = kNegInf;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t t = p * 16 + 4 * g16 + e;
      const bool valid = qvalid && t <= qpos;
      sv[e] = valid ? sacc[e] * scale : kNegInf;
      bad |= valid && !is_finite_f32(sv[e]);
      pm = fmaxf(pm, sv[e]);
    }
    pm = fmaxf(pm, __shfl_xor(pm, 16, 64));
    pm = fmaxf(pm, __shfl_xor(pm, 32, 64));
    const float m_new = fmaxf(m_run, pm);
    const float alpha = m_new == kNegInf ? 1.f : exp2_based(m_run - m_new);
    float ps = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float pe = sv[e] > kNegInf ? exp2_based(sv[e] - m_new) : 0.f;
      pbuf[wave][4 * g16 + e][j] = pe;
      ps += pe;
    }
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    l_run = l_run * alpha + ps;
    m_run = m_new;
    wave_lds_sync();

    // n = n alpha + P V over the page's 16 keys.
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), v));
      acc[v][0] *= a;
      acc[v][1] *= a;
    }
    const uint32_t* vt = reinterpret_cast<const uint32_t*>(&vtile[b][0][0]);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const uint32_t w = vt[k * 64 + lane];
      const float v0 = lo_bf16(w), v1 = hi_bf16(w);
      const float4* pk = reinterpret_cast<const float4*>(&pbuf[wave][k][0]);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float4 pq = pk[c];
        acc[4 * c + 0][0] = fmaf(pq.x, v0, acc[4 * c + 0][0]);
        acc[4 * c + 0][1] = fmaf(pq.x, v1, acc[4 * c + 0][1]);
        acc[4 * c + 1][0] = fmaf(pq.y, v0, acc[4 * c + 1][0]);
        acc[4 * c + 1][1] = fmaf(pq.y, v1, acc[4 * c + 1][1]);
        acc[4 * c + 2][0] = fmaf(pq.z, v0, acc[4 * c + 2][0]);
        acc[4 * c + 2][1] = fmaf(pq.z, v1, acc[4 * c + 2][1]);
        acc[4 * c + 3][0] = fmaf(pq.w, v0, acc[4 * c + 3][0]);
        acc[4 * c + 3][1] = fmaf(pq.w, v1, acc[4 * c + 3][1]);
      }
    }
  }

#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const uint32_t rv = wave * kRowsPerWave + v / G;
    if (rv < nrows) {
      const float L = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, l_run), v));
      const uint32_t o0 = f32_to_bf16(acc[v][0] / L), o1 = f32_to_bf16(acc[v][1] / L);
      bad |= !(L > 0.f) | ((o0 & 0x7f80u) == 0x7f80u) | ((o1 & 0x7f80u) == 0x7f80u);
      const uint32_t col = (h * G + v % G) * 128 + 2 * lane;
      const uint32_t word = o0 | (o1 << 16);
      if (out_mtiles)
        *reinterpret_cast<uint32_t*>(out + act_offset_m(row0 + rv, col, out_mtiles)) = word;
      else
        reinterpret_cast<uint32_t*>(out + ((uint64_t)(row0 + rv) * qh + h * G + v % G) * 128)[lane] = word;
    }
  }
  if (bad) raise_error(err, ERR_NONFINITE);
}

}  // namespace

uint32_t attention_block_rows(uint32_t qh, uint32_t kvh) { return 64u / (qh / kvh); }

hipError_t launch_attention_blocks(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                   const uint32_t* positions, const uint32_t* table, const uint32_t* blocks,
                                   uint32_t nblocks, uint16_t* out, uint32_t out_tiled, uint32_t out_rows,
                                   uint32_t qh, uint32_t kvh, uint32_t stride, uint32_t pages, uint32_t context,
                                   uint32_t* err, hipStream_t s) {
  if (nblocks == 0) return hipSuccess;
  const uint32_t mt = out_tiled ? act_mtiles(out_rows) : 0u;
  const dim3 grid(nblocks, kvh);
#define FH_BLOCKS(G_)                                                                                            \
  hipLaunchKernelGGL(attn_block_kernel<G_>, grid, dim3(256), 0, s, q, k_cache, v_cache, positions, table, blocks, \
                     out, mt, qh, kvh, stride, pages, context, err)
  switch (qh / kvh) {
    case 1: FH_BLOCKS(1); break;
    case 2: FH_BLOCKS(2); break;
    case 4: FH_BLOCKS(4); break;
    case 8: FH_BLOCKS(8); break;
    default: return hipErrorInvalidValue;
  }
#undef FH_BLOCKS
  return hipGetLastError();
}

}  // namespace fh
