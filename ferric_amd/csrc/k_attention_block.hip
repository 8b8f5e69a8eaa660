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
//   P V on v_mfma_f32_16x16x16bf16_1k. The score tile leaves lane (g, j)
//   holding P[vector j][keys 4 g .. 4 g + 3], which is that MFMA's A operand
//   as it stands. P is FP32; it enters as two bf16 terms, hi = bf16(p) and
//   lo = bf16(p - hi), whose sum is within 2^-17 p of p, and both products
//   are accumulated in FP32 (V is bf16, so every product is exact). V goes
//   through LDS transposed (dimension-major, two tokens per dword), so the B
//   operand of a lane (keys 4 g .. 4 g + 3 of one dimension) is two dwords.
// Finally out = bf16(n / l) for each valid row.
#include "common.hpp"
#include "kernels.hpp"

namespace fh {

namespace {

constexpr uint32_t kScaleBitsB = 0x3db504f3u;  // f32 1/sqrt(128), paged_decode.rs:31-35

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float exp2_based(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// V page in LDS, transposed: word [dim][pair] holds tokens 2 pair (low half)
// and 2 pair + 1 (high half) of one dimension; 9 words per dimension (8 and
// a pad) spread a wave's 64 stores over 16 banks.
constexpr int kVtPitch = 9;

template <int G>
__global__ __launch_bounds__(256, 4) void attn_block_kernel(
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
  __shared__ uint32_t vtile[2][128][kVtPitch];

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

  bool bad = false, bad_page = false;
  auto phys = [&](uint32_t pi) {
    uint32_t ph = pi < npages ? trow[pi] : 0u;
    if (ph >= pages) {
      bad_page = true;
      ph = 0;
    }
    return ph;
  };
  // K loader: thread t copies 16 bytes (dims 8 c .. 8 c + 7) of token t / 16.
  // V loader: wave w copies tokens 4 w .. 4 w + 3, one dword (dims 2 l,
  // 2 l + 1) per lane and token: a whole 256-byte row per load.
  const uint32_t lt = threadIdx.x >> 4, lc = threadIdx.x & 15;
  auto ksrc = [&](uint32_t ph) { return (((uint64_t)ph * 16 + lt) * kvh + h) * 128 + 8 * lc; };
  auto vsrc = [&](uint32_t ph, int t) {
    return reinterpret_cast<const uint32_t*>(vc + (((uint64_t)ph * 16 + 4 * wave + t) * kvh + h) * 128) + lane;
  };
  uint32_t ph_next = phys(1), ph_next2 = phys(2);
  u32x4 kreg;
  uint32_t vreg[4];
  {
    const uint32_t ph0 = phys(0);
    kreg = *reinterpret_cast<const u32x4*>(kc + ksrc(ph0));
#pragma unroll
    for (int t = 0; t < 4; ++t) vreg[t] = *vsrc(ph0, t);
  }

  const float scale = __builtin_bit_cast(float, kScaleBitsB);
  const float kNegInf = -__builtin_inff();
  float m_run = kNegInf, l_run = 0.f;
  // Output tiles, 16 dims each: lane l, element e holds vector 4 (l / 16) + e,
  // dim 16 d + l % 16.
  f32x4 acc[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Slots of the last page past the block's last position were never
  // written by this sequence and may hold any bits; their P is 0, but 0 times
  // a NaN or infinity inside the PV MFMA would still poison the sum, so they
  // enter as zeros (the reference never reads past the row's position).
  const uint32_t last_slot = pmax % 16;
  for (uint32_t p = 0; p < npages; ++p) {
    const int b = p & 1;
    ktile[b][lt][lc] = kreg;
    if (p + 1 == npages) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if ((uint32_t)(4 * wave + t) > last_slot) vreg[t] = 0u;
    }
    // Tokens (4 w, 4 w + 1) and (4 w + 2, 4 w + 3) -> pairs 2 w and 2 w + 1,
    // for dims 2 l (low halves) and 2 l + 1 (high halves).
#pragma unroll
    for (int pr = 0; pr < 2; ++pr) {
      const uint32_t t0 = vreg[2 * pr], t1 = vreg[2 * pr + 1];
      vtile[b][2 * lane][2 * wave + pr] = (t0 & 0xffffu) | (t1 << 16);
      vtile[b][2 * lane + 1][2 * wave + pr] = (t0 >> 16) | (t1 & 0xffff0000u);
    }
    if (p + 1 < npages) {
      kreg = *reinterpret_cast<const u32x4*>(kc + ksrc(ph_next));
#pragma unroll
      for (int t = 0; t < 4; ++t) vreg[t] = *vsrc(ph_next, t);
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
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float pe = sv[e] > kNegInf ? exp2_based(sv[e] - m_new) : 0.f;
      ps += pe;
      hi[e] = f32_to_bf16(pe);
      lo[e] = f32_to_bf16(pe - bf16_to_f32(hi[e]));
    }
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    l_run = l_run * alpha + ps;
    m_run = m_new;
    const uint32_t a_hi[2] = {hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16)};
    const uint32_t a_lo[2] = {lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16)};
    const bf16x4 p_hi = __builtin_bit_cast(bf16x4, a_hi), p_lo = __builtin_bit_cast(bf16x4, a_lo);

    // n = n alpha + P V: row e of this lane's output tiles is vector
    // 4 g16 + e, whose alpha lane 4 g16 + e computed.
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = __shfl(alpha, 4 * g16 + e, 64);
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[d][e] *= a;
    }
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const uint32_t* vt = &vtile[b][16 * d + j][2 * g16];
      const uint32_t bw[2] = {vt[0], vt[1]};
      const bf16x4 vb = __builtin_bit_cast(bf16x4, bw);
      acc[d] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(p_hi, vb, acc[d], 0, 0, 0);
      acc[d] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(p_lo, vb, acc[d], 0, 0, 0);
    }
  }

#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int v = 4 * g16 + e;
    const float L = __shfl(l_run, v, 64);
    const uint32_t rv = wave * kRowsPerWave + v / G;
    if (rv < nrows) {
      bad |= !(L > 0.f);
      const uint32_t head = h * G + v % G;
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const uint32_t o = f32_to_bf16(acc[d][e] / L);
        bad |= (o & 0x7f80u) == 0x7f80u;
        const uint32_t col = head * 128 + 16 * d + j;
        if (out_mtiles)
          out[act_offset_m(row0 + rv, col, out_mtiles)] = (uint16_t)o;
        else
          out[((uint64_t)(row0 + rv) * qh + head) * 128 + 16 * d + j] = (uint16_t)o;
      }
    }
  }
  if (bad) raise_error(err, ERR_NONFINITE);
  if (bad_page) raise_error(err, ERR_PAGE);
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
