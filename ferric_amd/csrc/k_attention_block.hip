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
// Grid (block, KV head), 4 waves per page phase. A wave owns 16 query
// vectors: 16 / G rows times the G query heads of the KV head (vector j: row
// j / G, head j % G). With PH page phases (PH groups of 4 waves, for grids
// too small to give every SIMD more than one wave, such as a speculative
// verify's few short blocks), phase f walks pages f, f + PH, f + 2 PH, ...
// and the phases' softmax states are folded pairwise through LDS at the end
// (m = max, the other terms scaled by exp(m_f - m)). Per 16-token page,
// shared by the phase's 4 waves through LDS (double-buffered, the next
// page's loads in flight while this one is used):
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
//
// QKN: the QK-norm, RoPE and KV append of the block's rows run here instead
// of in the QK-norm kernel (used when no block reads a slot another block of
// the chunk writes). The waves form the rows' G query heads, key head and
// value head from the QKV projection's split-K slabs with the QK-norm
// kernel's routine and order (bit-identical), keep them in LDS, write the key
// and value into the rows' cache slots, and use the LDS copies wherever a
// page holds one of those slots.
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

// LDS of a workgroup: per phase a double-buffered K tile and V tile; after
// the page loop the same bytes hold the phase states being folded, one slot
// per (phase pair, row group): 8 accumulator tiles of 64 lanes, then m and l
// of 16 vectors.
template <int PH>
struct BlockLds {
  static constexpr size_t kK = sizeof(u32x4) * PH * 2 * 16 * 17;
  static constexpr size_t kV = sizeof(uint32_t) * PH * 2 * 128 * kVtPitch;
  static constexpr size_t kSlot = sizeof(f32x4) * 8 * 64 + 2 * 16 * sizeof(float);
  static constexpr size_t kStage = PH > 1 ? (PH / 2) * 4 * kSlot : 0;
  static constexpr size_t kBytes = kK + kV > kStage ? kK + kV : kStage;
};

// Split-K slabs the fused QK-norm folds at most (all requested at once).
constexpr uint32_t kBlockQknMaxSplits = 8;

template <int G, int PH, bool QKN>
__global__ __launch_bounds__(256 * PH, 4) void attn_block_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    const uint32_t* __restrict__ positions, const uint32_t* __restrict__ table, const uint32_t* __restrict__ blocks,
    uint16_t* __restrict__ out, uint32_t out_mtiles, uint32_t qh, uint32_t kvh, uint32_t stride, uint32_t pages,
    uint32_t context, uint32_t* err, AttnQkn qk) {
  constexpr int kRowsPerWave = 16 / G;
  constexpr int kBlockRows = 64 / G;
  static_assert(16 % G == 0, "16 query vectors per wave");
  static_assert(PH == 1 || PH == 2 || PH == 4, "page phases");
  const uint32_t desc = blocks[blockIdx.x];
  const uint32_t row0 = desc & 0xffffu, nrows = desc >> 16;
  const uint32_t h = blockIdx.y;
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wave = PH == 1 ? w : w & 3, phase = PH == 1 ? 0 : w >> 2;  // row group within the phase, page phase
  const uint32_t last = row0 + nrows - 1;
  const uint32_t* trow = table + (uint64_t)last * stride;
  // The phase's first three page-table entries are requested with the
  // position (entries past the sequence's pages are checked once npages is
  // known), so the first K/V loads wait for one round trip, not two.
  uint32_t tpre[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) tpre[i] = trow[min((uint32_t)(phase + i * PH), stride - 1)];
  // Rows of a block have consecutive positions. A position past the context
  // or the page table is reported and the block reads page 0 only, with no
  // branch that the table loads above would be moved behind.
  const uint32_t pos_last = positions[last];
  const bool pos_ok = pos_last < context && pos_last / 16 < stride;
  if (!pos_ok && h == 0 && threadIdx.x == 0) raise_error(err, ERR_POSITION);
  const uint32_t pmax = pos_ok ? pos_last : 0u;
  const uint32_t npages = pmax / 16 + 1;

  __shared__ __attribute__((aligned(16))) unsigned char lds_raw[BlockLds<PH>::kBytes];
  auto ktile = reinterpret_cast<u32x4(*)[16][17]>(lds_raw + BlockLds<PH>::kK / PH * phase);
  auto vtile = reinterpret_cast<uint32_t(*)[128][kVtPitch]>(lds_raw + BlockLds<PH>::kK + BlockLds<PH>::kV / PH * phase);

  const int j = lane & 15, g16 = lane >> 4;
  // With page phases, a row group past the block's rows only helps load the
  // pages (one phase runs the wave's arithmetic as it is: masked rows).
  const bool live = PH == 1 || (uint32_t)(wave * kRowsPerWave) < nrows;
  const uint32_t rj = wave * kRowsPerWave + j / G;
  const bool qvalid = rj < nrows;
  const uint32_t qpos = qvalid ? positions[row0 + rj] : 0u;
  u32x4 qv[4];
  if constexpr (!QKN) {
    if (qvalid) {
      const uint16_t* qp = q + ((uint64_t)(row0 + rj) * qh + h * G + j % G) * 128 + 8 * g16;
#pragma unroll
      for (int i = 0; i < 4; ++i) qv[i] = *reinterpret_cast<const u32x4*>(qp + 32 * i);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) qv[i] = u32x4{0u, 0u, 0u, 0u};
    }
  }

  bool bad = false, bad_page = false;
  auto checked = [&](uint32_t pi, uint32_t ph) {
    ph = pi < npages ? ph : 0u;
    if (ph >= pages) {
      bad_page = true;
      ph = 0;
    }
    return ph;
  };
  auto phys = [&](uint32_t pi) { return checked(pi, pi < npages ? trow[pi] : 0u); };
  // K loader: thread t copies 16 bytes (dims 8 c .. 8 c + 7) of token t / 16.
  // V loader: wave w copies tokens 4 w .. 4 w + 3, one dword (dims 2 l,
  // 2 l + 1) per lane and token: a whole 256-byte row per load.
  const uint32_t lt = (threadIdx.x & 255) >> 4, lc = threadIdx.x & 15;
  auto ksrc = [&](uint32_t ph) { return (((uint64_t)ph * 16 + lt) * kvh + h) * 128 + 8 * lc; };
  auto vsrc = [&](uint32_t ph, int t) {
    return reinterpret_cast<const uint32_t*>(vc + (((uint64_t)ph * 16 + 4 * wave + t) * kvh + h) * 128) + lane;
  };
  uint32_t ph_next = checked(phase + PH, tpre[1]), ph_next2 = checked(phase + 2 * PH, tpre[2]);
  u32x4 kreg = u32x4{0u, 0u, 0u, 0u};
  uint32_t vreg[4] = {0u, 0u, 0u, 0u};
  if (PH == 1 || (uint32_t)phase < npages) {
    const uint32_t ph0 = checked(phase, tpre[0]);
    kreg = *reinterpret_cast<const u32x4*>(kc + ksrc(ph0));
#pragma unroll
    for (int t = 0; t < 4; ++t) vreg[t] = *vsrc(ph0, t);
  }

  // Fused QK-norm (QKN): the block's rows' heads, formed while the first
  // pages are in flight. Row i of the block holds position pos0 + i.
  __shared__ __attribute__((aligned(16))) uint16_t qkn_q[QKN ? kBlockRows * G * 128 : 1];
  __shared__ __attribute__((aligned(16))) uint16_t qkn_k[QKN ? kBlockRows * 128 : 1];
  __shared__ __attribute__((aligned(16))) uint16_t qkn_v[QKN ? kBlockRows * 128 : 1];
  // A round's squares (head-row slot, element) and their serial sums.
  __shared__ float qkn_sq[QKN ? 2 * 4 * PH : 1][QKN ? 129 : 1];
  __shared__ float qkn_sum[QKN ? 2 * 4 * PH : 1];
  uint32_t pos0 = 0;
  if constexpr (QKN) {
    pos0 = positions[row0];
    const uint32_t ld = (qh + 2 * kvh) * 128;
    const uint64_t slab = (uint64_t)qk.slab_rows * ld;
    const uint32_t nwork = nrows * (G + 2);
    // Each wave forms head-rows w, w + W, w + 2 W, ... (W waves), two at a
    // time with every load of both in flight together. A head-row is (row i,
    // role): roles 0..G-1 the query heads h G + role, G the key head and
    // G + 1 the value head of KV head h.
    constexpr uint32_t kWaves = 4 * PH;
    const uint32_t rounds = (nwork + 2 * kWaves - 1) / (2 * kWaves);  // uniform: the loop holds barriers
    for (uint32_t rd = 0; rd < rounds; ++rd) {
      const uint32_t hr0 = rd * 2 * kWaves + w;
      uint32_t hrs[2], rows_u[2], roles[2], pos[2];
      float pa[2][kBlockQknMaxSplits], pb[2][kBlockQknMaxSplits];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        hrs[u] = min(hr0 + u * kWaves, nwork - 1);  // a second past the end re-reads the last (not stored)
        const uint32_t i = hrs[u] / (G + 2);
        roles[u] = hrs[u] % (G + 2);
        rows_u[u] = row0 + i;
        pos[u] = positions[rows_u[u]];
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint32_t role = roles[u];
        const uint32_t head = role < (uint32_t)G ? h * G + role : (role == (uint32_t)G ? qh + h : qh + kvh + h);
        const float* pp = qk.qkv_part + (uint64_t)rows_u[u] * ld + head * 128 + lane;
        // Every slab load is unconditional (indices past the last slab
        // re-read it), so none waits in a branch; the sum takes the splits.
#pragma unroll
        for (uint32_t sp = 0; sp < kBlockQknMaxSplits; ++sp) {
          const uint64_t off = (uint64_t)min(sp, qk.splits - 1) * slab;
          pa[u][sp] = pp[off];
          pb[u][sp] = pp[off + 64];
        }
      }
      uint32_t page[2], wa[2], wb[2];
      float c[2], sn[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        page[u] = table[(uint64_t)rows_u[u] * stride + min(pos[u] / 16, stride - 1)];
        const uint16_t* wn = roles[u] < (uint32_t)G ? qk.q_norm : qk.k_norm;
        wa[u] = wn[lane];
        wb[u] = wn[lane + 64];
        const uint32_t trig = (pos[u] < context ? pos[u] : 0) * 64 + lane;
        c[u] = qk.cos_t[trig];
        sn[u] = qk.sin_t[trig];
      }
      // h = (P_0 + P_1 + ...) in split order, rounded once (the QK-norm
      // kernel's order). The squares go to LDS, and one lane per head-row
      // adds its 128 squares in element order (the wave routine's serial
      // sum, with no chain of lane reads), then the wave finishes the head.
      float fa[2], fb[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float a = pa[u][0], bsum = pb[u][0];
#pragma unroll
        for (uint32_t sp = 1; sp < kBlockQknMaxSplits; ++sp) {
          if (sp < qk.splits) {
            a += pa[u][sp];
            bsum += pb[u][sp];
          }
        }
        fa[u] = round_bf16(a);
        fb[u] = round_bf16(bsum);
        const int slot = w + u * kWaves;
        qkn_sq[slot][lane] = fa[u] * fa[u];
        qkn_sq[slot][64 + lane] = fb[u] * fb[u];
      }
      __syncthreads();
      if (threadIdx.x < 2 * kWaves) {
        float sum = 0.f;
#pragma unroll 16
        for (int l = 0; l < 128; ++l) sum = sum + qkn_sq[threadIdx.x][l];
        qkn_sum[threadIdx.x] = sum;
      }
      __syncthreads();
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        if (hr0 + u * kWaves >= nwork) break;
        const uint32_t role = roles[u], i = rows_u[u] - row0, pu = pos[u];
        const bool slot_ok = pu < context && pu / 16 < stride && page[u] < pages;
        if (!slot_ok && h == 0 && role == 0 && lane == 0) raise_error(err, ERR_PAGE);
        uint32_t ra, rb;
        if (role == (uint32_t)G + 1) {
          ra = f32_to_bf16(fa[u]);  // the value head: raw
          rb = f32_to_bf16(fb[u]);
        } else {
          bad |= qknorm_rope_wave_head_from_sum(fa[u], fb[u], qkn_sum[w + u * kWaves], bf16_to_f32(wa[u]),
                                                bf16_to_f32(wb[u]), c[u], sn[u], qk.eps, ra, rb);
        }
        uint16_t* ls =
            role < (uint32_t)G ? qkn_q + (i * G + role) * 128 : (role == (uint32_t)G ? qkn_k : qkn_v) + i * 128;
        ls[lane] = (uint16_t)ra;
        ls[lane + 64] = (uint16_t)rb;
        if (role >= (uint32_t)G && slot_ok) {
          uint16_t* dst = (role == (uint32_t)G ? qk.k_cache : qk.v_cache) +
                          (((uint64_t)page[u] * 16 + (pu & 15u)) * kvh + h) * 128;
          dst[lane] = (uint16_t)ra;
          dst[lane + 64] = (uint16_t)rb;
        }
      }
    }
    __syncthreads();
    if (qvalid) {
      const uint16_t* qp = qkn_q + (rj * G + j % G) * 128 + 8 * g16;
#pragma unroll
      for (int i = 0; i < 4; ++i) qv[i] = *reinterpret_cast<const u32x4*>(qp + 32 * i);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) qv[i] = u32x4{0u, 0u, 0u, 0u};
    }
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
  const uint32_t iters = (npages + PH - 1) / PH;
  // One iteration: every phase's next page. Only the last iteration (LAST)
  // can hold the block's last page or find a phase with no page left, and it
  // issues no loads, so the loop before it runs without those branches.
  auto step = [&](uint32_t it, auto last_tag) {
    constexpr bool LAST = decltype(last_tag)::value;
    const uint32_t p = phase + it * PH;
    const bool here = !LAST || PH == 1 || p < npages;  // the phase has a page this iteration
    const int b = it & 1;
    if (here) {
      if constexpr (QKN) {
        // The block's own new slots (positions pos0 .. pmax) come from LDS.
        if (p * 16 + 15 >= pos0) {
          const uint32_t tk = p * 16 + lt;
          if (tk >= pos0 && tk <= pmax) kreg = *reinterpret_cast<const u32x4*>(qkn_k + (tk - pos0) * 128 + 8 * lc);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const uint32_t tv = p * 16 + 4 * wave + t;
            if (tv >= pos0 && tv <= pmax) vreg[t] = reinterpret_cast<const uint32_t*>(qkn_v + (tv - pos0) * 128)[lane];
          }
        }
      }
      ktile[b][lt][lc] = kreg;
      if (LAST && p + 1 == npages) {
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
      if (!LAST && (PH == 1 || p + PH < npages)) {
        kreg = *reinterpret_cast<const u32x4*>(kc + ksrc(ph_next));
#pragma unroll
        for (int t = 0; t < 4; ++t) vreg[t] = *vsrc(ph_next, t);
      }
    }
    if (!LAST) {
      ph_next = ph_next2;
      ph_next2 = phys(p + 3 * PH);
    }
    __syncthreads();
    if (!here || !live) return;

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
  };
  for (uint32_t it = 0; it + 1 < iters; ++it) step(it, std::false_type{});
  step(iters - 1, std::true_type{});

  if constexpr (PH > 1) {
    // Fold the phases pairwise: in the first round phase f + PH / 2 hands its
    // state to phase f through slot f; in later rounds phase f + half hands
    // it through slot f + half (which only that phase read before).
    f32x4* st_acc = reinterpret_cast<f32x4*>(lds_raw);
    float* st_ml = reinterpret_cast<float*>(lds_raw + sizeof(f32x4) * (PH / 2) * 4 * 8 * 64);
    __syncthreads();  // every wave is done with the page tiles
#pragma unroll
    for (int half = PH / 2; half >= 1; half /= 2) {
      const bool first = 2 * half == PH;
      if (live && phase >= half && phase < 2 * half) {
        const int slot = (first ? phase - half : phase) * 4 + wave;
#pragma unroll
        for (int d = 0; d < 8; ++d) st_acc[(slot * 8 + d) * 64 + lane] = acc[d];
        if (g16 == 0) {
          st_ml[slot * 32 + j] = m_run;
          st_ml[slot * 32 + 16 + j] = l_run;
        }
      }
      __syncthreads();
      if (live && phase < half) {
        const int slot = (first ? phase : phase + half) * 4 + wave;
        const float mo = st_ml[slot * 32 + j], lo = st_ml[slot * 32 + 16 + j];
        const float m_new = fmaxf(m_run, mo);
        const float a_self = m_run == kNegInf ? 0.f : exp2_based(m_run - m_new);
        const float a_other = mo == kNegInf ? 0.f : exp2_based(mo - m_new);
        l_run = l_run * a_self + lo * a_other;
        m_run = m_new;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float fs = __shfl(a_self, 4 * g16 + e, 64), fo = __shfl(a_other, 4 * g16 + e, 64);
#pragma unroll
          for (int d = 0; d < 8; ++d) acc[d][e] = acc[d][e] * fs + st_acc[(slot * 8 + d) * 64 + lane][e] * fo;
        }
      }
    }
  }

#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int v = 4 * g16 + e;
    const float L = __shfl(l_run, v, 64);
    const uint32_t rv = wave * kRowsPerWave + v / G;
    if (phase == 0 && rv < nrows) {  // phase 0 holds the folded state
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
                                   uint32_t* err, hipStream_t s, const AttnQkn* qkn) {
  if (nblocks == 0) return hipSuccess;
  if (qkn && !attention_blocks_qkn_supported(qh, kvh, qkn->splits)) return hipErrorInvalidValue;
  const uint32_t mt = out_tiled ? act_mtiles(out_rows) : 0u;
  const dim3 grid(nblocks, kvh);
  const AttnQkn qa = qkn ? *qkn : AttnQkn{};
  // Page phases so that a small grid still puts about four waves on each
  // SIMD (256 CUs): a workgroup of 4 PH waves per block and head.
  const uint64_t wgs = (uint64_t)nblocks * kvh;
  const int ph = wgs <= 256 ? 4 : wgs <= 512 ? 2 : 1;
#define FH_BLOCKS_PH(G_, PH_, QKN_)                                                                               \
  hipLaunchKernelGGL((attn_block_kernel<G_, PH_, QKN_>), grid, dim3(256 * PH_), 0, s, q, k_cache, v_cache,        \
                     positions, table, blocks, out, mt, qh, kvh, stride, pages, context, err, qa)
#define FH_BLOCKS_Q(G_, QKN_)      \
  if (ph == 4)                     \
    FH_BLOCKS_PH(G_, 4, QKN_);     \
  else if (ph == 2)                \
    FH_BLOCKS_PH(G_, 2, QKN_);     \
  else                             \
    FH_BLOCKS_PH(G_, 1, QKN_)
#define FH_BLOCKS(G_)        \
  if (qkn) {                 \
    FH_BLOCKS_Q(G_, true);   \
  } else {                   \
    FH_BLOCKS_Q(G_, false);  \
  }
  switch (qh / kvh) {
    case 1: FH_BLOCKS(1); break;
    case 2: FH_BLOCKS(2); break;
    case 4: FH_BLOCKS(4); break;
    case 8: FH_BLOCKS_Q(8, false); break;
    default: return hipErrorInvalidValue;
  }
#undef FH_BLOCKS
#undef FH_BLOCKS_Q
#undef FH_BLOCKS_PH
  return hipGetLastError();
}

bool attention_blocks_qkn_supported(uint32_t qh, uint32_t kvh, uint32_t qkv_splits) {
  return kvh && qh % kvh == 0 && qh / kvh <= 4 && (qh / kvh & (qh / kvh - 1)) == 0 && qkv_splits >= 1 &&
         qkv_splits <= kBlockQknMaxSplits;
}

}  // namespace fh
