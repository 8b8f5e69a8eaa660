// K4 paged GQA decode attention for gfx950: split-context partitions with an
// ordered merge.
//
// Reference semantics (device/qwen3-all-kernels-v1/src/paged_decode.rs:222-572):
// for a query row at position p, keys t = 0..p through the row's page table,
// score = (q . k_t) * f32(0x3db504f3), softmax, out = bf16(n / l). The
// reference's split variant (device/qwen3-tp-c1-split8-attention-kernels-v21,
// README.md:42-80) partitions the context, keeps an FP32 state (m, l, n[128])
// per partition, merges the partitions in ascending order, then divides and
// narrows once. These kernels keep that contract with 16- or 32-page
// partitions (attn_split_pages).
//
// K and V are read once per step, so their loads are non-temporal: letting
// them allocate in the caches cost about 13% of the kernel's time (measured
// with 32 rows of mean context 4K, 550 MB of K/V per layer).
//
// Partition kernel, grid (partition, KV head, row), 8 waves; each wave takes
// PP / 8 of the partition's PP pages and the G query heads of the KV head, so
// every K/V byte is read once per token row. A wave makes two memory round
// trips, each with all of its pages' loads in flight at once:
//   1. K: whole 256-byte token rows per load, re-laid through a padded LDS
//      tile into the MFMA A operand (lane l: token l % 16, dims 32 i + 8 (l/16)
//      for MFMA i); S^T = K Q^T on v_mfma_f32_16x16x32_bf16 with the G queries
//      as the B operand; scaled, masked scores go to LDS.
//   2. V loads issued as soon as the scores are out, in flight during the
//      exact softmax over the wave's 64 tokens (max, p = exp(s - max), sum);
//      then PV on VALU: lane l owns output dims 2l, 2l+1, and a token's V row
//      is one coalesced 256-byte wave load.
// The eight wave states (m, l, n[128]) are merged in wave order. A row whose
// context fits one partition is finished here (divide, narrow, store);
// longer rows leave partition states, merged either by the merge kernel or,
// in the fused form, by the partition workgroup of each (row, KV head) that
// finishes last (a per-pair arrival counter; it resets the counter).
// Merge (merge_records, in either kernel): partition weights
// w_p = exp(m_p - M) with M the maximum over partitions, then l and n are
// summed over partitions in ascending order, divided, narrowed once. Both
// forms run the same code on the same records, so their outputs are equal.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

// The in-kernel merge (FUSED) publishes partition records with relaxed
// agent-scope atomic stores, waits for them (s_waitcnt), then counts the
// workgroup in with a relaxed atomic; the last workgroup reads the records
// with relaxed agent-scope atomic loads. There is no release/acquire pair:
// correctness rests on how gfx950 lowers these operations (stores written
// through the XCD's L2 with sc1, loads that bypass it, and a wait that
// covers store completion), so this file is built for gfx950 only.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "k_attention.hip: the in-kernel partition merge is written for gfx950's memory-model lowering"
#endif

namespace fh {

namespace {

constexpr int kAttnThreads = 256;
constexpr uint32_t kScaleBits = 0x3db504f3u;  // f32 1/sqrt(128), paged_decode.rs:31-35

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// e^x as 2^(x log2 e) on the hardware exp2 (v_exp_f32, about 1 ulp). The
// reference uses the library expf; the softmax terms it feeds are compared
// to tolerance, and the relative difference here is below 1e-6 for the
// |x| < 100 that a max-subtracted softmax sees. exp(-inf) = 0 as required.
__device__ __forceinline__ float exp_fast(float x) {
  return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}

// Stores one finished head output (dims 2*lane, 2*lane+1) in either layout.
// Row r of the launch is row row0 + r of the output; the tiled layout has
// out_mtiles row tiles (0: row-major [rows][qh * 128]).
__device__ __forceinline__ void store_head(uint16_t* out, uint32_t out_mtiles, uint32_t row0, uint32_t r, uint32_t qh,
                                          uint32_t head, int lane, uint32_t o0, uint32_t o1) {
  const uint32_t col = head * 128 + 2 * lane;
  const uint32_t word = o0 | (o1 << 16);
  if (out_mtiles)
    *reinterpret_cast<uint32_t*>(out + act_offset_m(row0 + r, col, out_mtiles)) = word;
  else
    reinterpret_cast<uint32_t*>(out + ((uint64_t)(row0 + r) * qh + head) * 128)[lane] = word;
}

// Merges the ns partition records at p (one (row, query head), records of
// kAttnPartialFloats floats) in ascending partition order; this lane's
// output dims 2 lane, 2 lane + 1 come back unnormalised in n0, n1 with the
// denominator L.
template <bool COHERENT = false>
__device__ __forceinline__ float load_record(const float* p) {
  if constexpr (COHERENT)
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    return *p;
}

// COHERENT: every record load is an agent-scope atomic load (records written
// in the same launch by workgroups on other XCDs, see the partition kernel).
constexpr uint32_t kMergeInFlight = 16;
template <bool COHERENT = false>
__device__ __forceinline__ void merge_records(const float* p, uint32_t ns, int lane, float& L, float& n0,
                                              float& n1) {
  const float kNegInf = -__builtin_inff();
  if (ns <= kMergeInFlight) {
    // Up to 16 partitions: every record's m and l (lane s: partition s) and
    // this lane's two numerators of every record are requested at once, one
    // memory round trip; then the arithmetic below in the same order. The
    // loads are unconditional (indices past the last record re-read it) so
    // that none sits in a branch whose join would wait for it.
    const bool own = (uint32_t)lane < ns;
    const float* pl = p + (uint64_t)min((uint32_t)lane, ns - 1) * kAttnPartialFloats;
    const float m_raw = load_record<COHERENT>(pl);
    const float l_raw = load_record<COHERENT>(pl + 1);
    float a0[kMergeInFlight], a1[kMergeInFlight];
#pragma unroll
    for (uint32_t u = 0; u < kMergeInFlight; ++u) {
      const float* ps = p + (uint64_t)min(u, ns - 1) * kAttnPartialFloats;
      a0[u] = load_record<COHERENT>(ps + 2 + 2 * lane);
      a1[u] = load_record<COHERENT>(ps + 3 + 2 * lane);
    }
    const float ms = own ? m_raw : kNegInf;
    const float ls = own ? l_raw : 0.f;
    const float M = wave_max(ms);
    const float ws = own ? expf(ms - M) : 0.f;
    const float lw = own ? ls * ws : 0.f;
    L = 0.f;
    n0 = 0.f;
    n1 = 0.f;
#pragma unroll
    for (uint32_t u = 0; u < kMergeInFlight; ++u) {
      if (u < ns) {
        const float w = lane_bcast(ws, (int)u);
        L += lane_bcast(lw, (int)u);
        n0 += a0[u] * w;
        n1 += a1[u] * w;
      }
    }
    return;
  }
  float mloc = kNegInf;
  for (uint32_t sp = lane; sp < ns; sp += 64) mloc = fmaxf(mloc, load_record<COHERENT>(p + (uint64_t)sp * kAttnPartialFloats));
  const float M = wave_max(mloc);
  L = 0.f;
  n0 = 0.f;
  n1 = 0.f;
  for (uint32_t c0 = 0; c0 < ns; c0 += 64) {
    // Lane s holds partition c0 + s's weight exp(m - M) and weighted l.
    const uint32_t mine = c0 + lane;
    const float ms = mine < ns ? load_record<COHERENT>(p + (uint64_t)mine * kAttnPartialFloats) : kNegInf;
    const float ws = mine < ns ? expf(ms - M) : 0.f;
    const float lw = mine < ns ? load_record<COHERENT>(p + (uint64_t)mine * kAttnPartialFloats + 1) * ws : 0.f;
    const uint32_t cn = min(64u, ns - c0);
    for (uint32_t s0 = 0; s0 < cn; s0 += 8) {
      // Eight partitions' numerators in flight, then added in ascending order.
      float a0[8], a1[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const uint32_t sp = s0 + u;
        const float* ps = p + (uint64_t)(c0 + sp) * kAttnPartialFloats;
        a0[u] = sp < cn ? load_record<COHERENT>(ps + 2 + 2 * lane) : 0.f;
        a1[u] = sp < cn ? load_record<COHERENT>(ps + 3 + 2 * lane) : 0.f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const uint32_t sp = s0 + u;
        if (sp < cn) {
          const float w = lane_bcast(ws, (int)sp);
          L += lane_bcast(lw, (int)sp);
          n0 += a0[u] * w;
          n1 += a1[u] * w;
        }
      }
    }
  }
}

// One workgroup per (partition, KV head, row); its WAVES waves split the
// partition's PP pages (PP / WAVES each) and serve the G query heads of the
// KV head. A wave issues all of its K loads at once, scores them, then
// issues all of its V loads at once: two memory round trips per wave.
// FUSED: counters[r * kvh + h] counts the finished partitions of a
// multi-partition (row, KV head); the one that finishes last merges.
// QKS > 0: the QK-norm + RoPE + KV append stage runs here (AttnQkn): q is
// formed from QKS split-K slabs of the QKV projection instead of read from
// `q`, and the new token's K/V are formed, appended and used in place of
// the cache's slot.
template <int G, int WAVES, int PP, bool FUSED, int QKS>
__global__ __launch_bounds__(WAVES * 64) void attn_partition_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    const uint32_t* __restrict__ positions, const uint32_t* __restrict__ table, float* __restrict__ part,
    uint16_t* __restrict__ out, uint32_t out_mtiles, uint32_t row0, uint32_t qh, uint32_t kvh, uint32_t stride,
    uint32_t pages, uint32_t context, uint32_t smax, uint32_t* counters, uint32_t* err, AttnQkn qk) {
  constexpr uint32_t kWavePages = PP / WAVES;
  static_assert(PP % WAVES == 0 && kWavePages >= 1, "pages split evenly over the waves");
  constexpr bool kQkn = QKS > 0;
  static_assert(!kQkn || G + 2 <= WAVES, "one wave per query head, one for the key and one for the value head");
  // With at most two pages per wave the V registers fit beside K's, so V is
  // requested together with K (one memory round trip instead of two). Not
  // for G = 2 (Qwen3-0.6B), whose partitions would drop from 3 to 2
  // workgroups per CU with the extra registers.
  constexpr bool kEarlyV = kQkn && kWavePages <= 2 && G >= 4;
  const uint32_t split = blockIdx.x, h = blockIdx.y, r = blockIdx.z;
  // The wave index is uniform; saying so keeps every page address scalar.
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t p0 = split * PP;

  // This wave's pages: [w0, w0 + np) of the row. The page-table entries are
  // requested together with the position (they do not depend on it), so the
  // K loads wait for one memory round trip, not two.
  const uint32_t w0 = p0 + wave * kWavePages;
  const uint32_t* trow = table + (uint64_t)r * stride;
  static_assert(kWavePages <= 64, "one page-table entry per lane");
  const uint32_t raw_phys = lane < (int)kWavePages && w0 + lane < stride ? trow[w0 + lane] : 0u;
  const uint32_t pos = positions[r];
  __builtin_amdgcn_sched_barrier(0);

  // Fused QK-norm, part 1. Wave w < G forms query head h G + w, wave G the
  // key head and wave G + 1 the value head of KV head h (lane l: elements l
  // and l + 64). Their slab and norm-weight loads go out right after the
  // position and page-table loads and before the K loads: a wave's loads
  // complete in issue order, so the K addresses (which need the position)
  // do not wait for the slabs, and anything requested after the K loads
  // could only be used once K has landed.
  const int qk_role = kQkn && wave < G + 2 ? wave : -1;
  float qk_a[kQkn ? QKS : 1], qk_b[kQkn ? QKS : 1];
  uint32_t qk_wa = 0u, qk_wb = 0u;
  if constexpr (kQkn) {
    // Every wave issues these (the ones without a head re-read query head
    // h G): loads under a branch would be joined with the branch's other
    // side right here, which makes the wave wait for them.
    const int role = qk_role >= 0 ? qk_role : 0;
    const uint32_t ld = (qh + 2 * kvh) * 128;
    const uint32_t head = role < G ? h * G + role : (role == G ? qh + h : qh + kvh + h);
    const float* pp = qk.qkv_part + (uint64_t)r * ld + head * 128 + lane;
    const uint64_t slab = (uint64_t)qk.slab_rows * ld;
#pragma unroll
    for (int sp = 0; sp < QKS; ++sp) {
      qk_a[sp] = pp[sp * slab];
      qk_b[sp] = pp[sp * slab + 64];
    }
    const uint16_t* wn = role < G ? qk.q_norm : qk.k_norm;  // (the value head's go unused)
    qk_wa = wn[lane];  // widened where used: converting here would wait for the load
    qk_wb = wn[lane + 64];
  }
  __builtin_amdgcn_sched_barrier(0);
  if (pos >= context || pos / 16 >= stride) {
    // (The separate QK-norm kernel reports this row's missing KV slot as a
    // page fault; the fused form reports both.)
    if (split == 0 && h == 0 && threadIdx.x == 0) raise_error(err, kQkn ? (ERR_POSITION | ERR_PAGE) : ERR_POSITION);
    return;
  }
  const uint32_t ctx = pos + 1;
  const uint32_t row_pages = (ctx + 15) / 16;
  if (p0 >= row_pages) return;  // uniform per workgroup
  const uint32_t nsplit = (row_pages + PP - 1) / PP;
  const uint32_t np = w0 < row_pages ? min(row_pages - w0, kWavePages) : 0u;
  // Fused: the last partition holds the new token (page pos / 16, slot
  // pos % 16); the wave whose pages include it appends and uses the new K/V.
  const bool last_part = split == nsplit - 1;
  const uint32_t upos = pos / 16 - w0;  // page index within this wave when it owns the token
  const bool own_pos = kQkn && last_part && pos / 16 >= w0 && upos < np;
  const uint32_t epos = pos & 15u;

  // Scores of the wave's tokens, replaced in place by probabilities: [token][g].
  __shared__ float sbuf[WAVES][kWavePages * 16][G];
  __shared__ float wstat[WAVES][2][G];
  __shared__ float wacc[WAVES][G][128];
  float* sw = &sbuf[wave][0][0];

  const int g16 = lane >> 4, r16 = lane & 15;
  const float scale = __builtin_bit_cast(float, kScaleBits);
  const float kNegInf = -__builtin_inff();
  bool bad = false;

  // B operand: query head h*G + r16 (zero for r16 >= G); MFMA i, lane group
  // g16 covers dims 32*i + 8*g16 .. +7.
  u32x4 qv[4];
  if constexpr (!kQkn) {
    if (r16 < G) {
      const uint16_t* qp = q + ((uint64_t)r * qh + h * G + r16) * 128 + 8 * g16;
#pragma unroll
      for (int i = 0; i < 4; ++i) qv[i] = *reinterpret_cast<const u32x4*>(qp + 32 * i);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) qv[i] = u32x4{0u, 0u, 0u, 0u};
    }
  }

  // Physical pages of this wave, one per lane, read back with readlane so no
  // scalar table load sits between page loads.
  uint32_t my_phys = lane < (int)np ? raw_phys : 0u;
  const bool bad_page = my_phys >= pages;  // an index fault, not a value fault
  if (bad_page) my_phys = 0;
  auto phys_of = [&](uint32_t j) { return (uint32_t)__builtin_amdgcn_readlane((int)my_phys, (int)j); };

  // Pass 1: S^T = K Q^T on MFMA per page, scaled and masked scores to LDS,
  // and each query head's maximum over the wave's tokens.
  const uint32_t vstride = kvh * 64;  // dwords between consecutive slots of one head
  uint32_t vd[kWavePages][16];
  // ALL: as load_k below.
  auto load_v = [&](auto all_tag) {
    constexpr bool ALL = decltype(all_tag)::value;
    const uint32_t spare = np ? phys_of(0) : 0u;
#pragma unroll
    for (uint32_t u = 0; u < kWavePages; ++u) {
      if (ALL || u < np) {
        const uint32_t pu = ALL && u >= np ? spare : phys_of(u);
        const uint32_t* vp = reinterpret_cast<const uint32_t*>(vc + (((uint64_t)pu * 16) * kvh + h) * 128) + lane;
#pragma unroll
        for (int e = 0; e < 16; ++e) vd[u][e] = __builtin_nontemporal_load(vp + e * vstride);
      }
    }
  };

  float pm = kNegInf;  // this lane's max for query column r16
  auto score_page = [&](uint32_t u, const u32x4 (&ka)[4]) {
    f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ka[i]),
                                                    __builtin_bit_cast(bf16x8, qv[i]), sacc, 0, 0, 0);
    // Lane holds query r16 for tokens 4*g16 + e of the page.
    const uint32_t t = u * 16 + 4 * g16;  // token within the wave's range
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool valid = w0 * 16 + t + e < ctx;
      const float sv = valid ? sacc[e] * scale : kNegInf;
      bad |= valid && !is_finite_f32(sv);
      pm = fmaxf(pm, sv);
      if (r16 < G) sw[(t + e) * G + r16] = sv;
    }
  };
  // Fused: the formed heads (bf16): query heads 0..G-1, then the new K and V.
  __shared__ __align__(16) uint32_t qkn_s[kQkn ? G + 2 : 1][64];
  {
    // Whole 256-byte token rows per load (lane: token 4 i + g16, dims
    // 8 r16 .. 8 r16 + 7), turned into the A-operand layout through a padded
    // LDS tile (272-byte rows keep the column reads conflict-free).
    __shared__ u32x4 ktile[WAVES][16][17];
    u32x4 kr[kWavePages][4];
    // ALL: issue a load for every page slot of the wave, pages past the
    // context re-reading the wave's first page (or page 0), so the number of
    // loads in flight is the same on every path and a wait for an earlier
    // load does not also wait for these.
    auto load_k = [&](auto all_tag) {
      constexpr bool ALL = decltype(all_tag)::value;
      const uint32_t spare = np ? phys_of(0) : 0u;
#pragma unroll
      for (uint32_t u = 0; u < kWavePages; ++u) {
        if (ALL || u < np) {
          const uint32_t pu = ALL && u >= np ? spare : phys_of(u);
          const uint16_t* kp = kc + (((uint64_t)pu * 16 + g16) * kvh + h) * 128 + 8 * r16;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            kr[u][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kp + (uint64_t)4 * i * kvh * 128));
        }
      }
    };
    if constexpr (kQkn) {
      if (qk_role >= 0) {
        // Fused QK-norm, part 2 (the decode QK-norm kernel's arithmetic, the
        // same routine): RoPE factors at the position, then this wave's K
        // (and V) loads, then fold the slabs in split order, round, and
        // normalize and rotate (query and key heads) or keep raw (value).
        const float qk_c = qk.cos_t[(uint64_t)pos * 64 + lane];
        const float qk_s = qk.sin_t[(uint64_t)pos * 64 + lane];
        load_k(std::true_type{});
        if constexpr (kEarlyV) load_v(std::true_type{});
        __builtin_amdgcn_sched_barrier(0);
        if (qk_role < G || last_part) {
          float a = qk_a[0], b = qk_b[0];
#pragma unroll
          for (int sp = 1; sp < QKS; ++sp) {
            a += qk_a[sp];
            b += qk_b[sp];
          }
          a = round_bf16(a);
          b = round_bf16(b);
          uint32_t ra, rb;
          if (qk_role <= G) {
            bad |= qknorm_rope_wave_head(a, b, bf16_to_f32(qk_wa), bf16_to_f32(qk_wb), qk_c, qk_s, qk.eps, ra, rb);
          } else {
            ra = f32_to_bf16(a);
            rb = f32_to_bf16(b);
          }
          uint16_t* row_s = reinterpret_cast<uint16_t*>(&qkn_s[qk_role][0]);
          row_s[lane] = (uint16_t)ra;
          row_s[lane + 64] = (uint16_t)rb;
        }
      } else {
        load_k(std::false_type{});
        if constexpr (kEarlyV) load_v(std::false_type{});
      }
      __syncthreads();
      if (r16 < G) {
        const uint16_t* qp = reinterpret_cast<const uint16_t*>(&qkn_s[r16][0]) + 8 * g16;
#pragma unroll
        for (int i = 0; i < 4; ++i) qv[i] = *reinterpret_cast<const u32x4*>(qp + 32 * i);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) qv[i] = u32x4{0u, 0u, 0u, 0u};
      }
      if (own_pos) {
        // Append the new token's K and V at (pages[pos / 16], pos % 16), as
        // the decode QK-norm kernel does (nothing is written to a page
        // outside the pool; that page is reported below).
        const uint32_t phys = __builtin_amdgcn_readlane((int)raw_phys, (int)upos);
        if (phys < pages) {
          const uint64_t slot = ((uint64_t)phys * 16 + epos) * kvh + h;
          reinterpret_cast<uint32_t*>(qk.k_cache + slot * 128)[lane] = qkn_s[G][lane];
          reinterpret_cast<uint32_t*>(qk.v_cache + slot * 128)[lane] = qkn_s[G + 1][lane];
        }
      }
    } else {
      load_k(std::false_type{});
    }
#pragma unroll
    for (uint32_t u = 0; u < kWavePages; ++u) {
      if (u < np) {
        if constexpr (kQkn) {
          // The new token's K replaces whatever its slot held.
          if (own_pos && u == upos) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (4 * i + g16 == (int)epos) kr[u][i] = *reinterpret_cast<const u32x4*>(&qkn_s[G][4 * r16]);
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) ktile[wave][4 * i + g16][r16] = kr[u][i];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        u32x4 ka[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) ka[i] = ktile[wave][r16][g16 + 4 * i];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        score_page(u, ka);
      }
    }
  }
  // V loads go out now, so they are in flight during the softmax.
  if constexpr (!kEarlyV) load_v(std::false_type{});
  pm = fmaxf(pm, __shfl_xor(pm, 16, 64));
  pm = fmaxf(pm, __shfl_xor(pm, 32, 64));
  float m[G], l[G], acc[G][2];
#pragma unroll
  for (int g = 0; g < G; ++g) m[g] = lane_bcast(pm, g);  // lanes with r16 = g hold head g's max
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // Probabilities p = exp(s - m) in place and the denominators l (per-lane
  // partial sums in ascending token order, then a fixed butterfly).
  const uint32_t ntok = np * 16;
  float ls[G];
#pragma unroll
  for (int g = 0; g < G; ++g) ls[g] = 0.f;
  for (uint32_t t = lane; t < ntok; t += 64) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float sv = sw[t * G + g];
      const float pv = sv > kNegInf ? exp_fast(sv - m[g]) : 0.f;
      sw[t * G + g] = pv;
      ls[g] += pv;
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    l[g] = wave_sum(ls[g]);
    acc[g][0] = acc[g][1] = 0.f;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // Pass 2: n += p * v on VALU; lane l owns output dims 2l, 2l+1, and a
  // token's V row is one coalesced 256-byte wave load.
  if constexpr (kQkn) {
    if (own_pos) {
      // The new token's V replaces whatever its slot held.
      const uint32_t vn = qkn_s[G + 1][lane];
#pragma unroll
      for (uint32_t u = 0; u < kWavePages; ++u)
        if (u == upos) {
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if ((uint32_t)e == epos) vd[u][e] = vn;
        }
    }
  }
  {
    auto pv_page = [&](auto full_tag, uint32_t u) {
      constexpr bool FULL = decltype(full_tag)::value;
      const uint32_t valid = FULL ? 16u : min(16u, ctx - (w0 + u) * 16);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t v = FULL || (uint32_t)e < valid ? vd[u][e] : 0u;  // slots past the context may hold anything
        const float v0 = lo_bf16(v), v1 = hi_bf16(v);
        const float* pt = sw + (u * 16 + e) * G;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float pg = pt[g];
          acc[g][0] = fmaf(pg, v0, acc[g][0]);
          acc[g][1] = fmaf(pg, v1, acc[g][1]);
        }
      }
    };
#pragma unroll
    for (uint32_t u = 0; u < kWavePages; ++u) {
      if (u < np) {
        if ((w0 + u + 1) * 16 <= ctx)
          pv_page(std::true_type{}, u);
        else
          pv_page(std::false_type{}, u);
      }
    }
  }

  // Merge the waves' states in wave order (waves past the context have l = 0).
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
    for (int g = wave; g < G; g += WAVES) {
      float M = wstat[0][0][g];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) M = fmaxf(M, wstat[w][0][g]);
      float L = 0.f, n0 = 0.f, n1 = 0.f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        const float lw = wstat[w][1][g];
        if (lw > 0.f) {
          const float f = exp_fast(wstat[w][0][g] - M);
          L += lw * f;
          n0 += wacc[w][g][2 * lane] * f;
          n1 += wacc[w][g][2 * lane + 1] * f;
        }
      }
      const uint32_t o0 = f32_to_bf16(n0 / L), o1 = f32_to_bf16(n1 / L);
      bad |= !(L > 0.f) | ((o0 & 0x7f80u) == 0x7f80u) | ((o1 & 0x7f80u) == 0x7f80u);
      store_head(out, out_mtiles, row0, r, qh, h * G + g, lane, o0, o1);
    }
  } else {
    // Partition state (m, l, n[128]) of each query head.
    for (int idx = threadIdx.x; idx < G * (int)kAttnPartialFloats; idx += WAVES * 64) {
      const int g = idx / (int)kAttnPartialFloats, c = idx % (int)kAttnPartialFloats;
      float M = wstat[0][0][g];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) M = fmaxf(M, wstat[w][0][g]);
      float v;
      if (c == 0) {
        v = M;
      } else {
        v = 0.f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
          const float lw = wstat[w][1][g];
          if (lw > 0.f) v += (c == 1 ? lw : wacc[w][g][c - 2]) * exp_fast(wstat[w][0][g] - M);
        }
      }
      float* dst = part + (((uint64_t)r * qh + h * G + g) * smax + split) * kAttnPartialFloats + c;
      if constexpr (FUSED)
        __hip_atomic_store(dst, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else
        *dst = v;
    }
    if constexpr (FUSED) {
      // The records are agent-scope atomic stores: the XCDs' L2 caches are
      // not coherent with each other, and an agent-scope fence per workgroup
      // (an L2 write-back and invalidate) costs more than the merge launch it
      // would save. Each thread waits for its stores to complete, then the
      // workgroup counts itself in; the workgroup that brings the count to
      // nsplit merges the pair's G heads with agent-scope atomic loads (the
      // merge kernel's code and order, so its outputs are the same).
      __shared__ uint32_t last_s;
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      uint32_t* counter = counters + (uint64_t)r * kvh + h;
      if (threadIdx.x == 0) last_s = atomicAdd(counter, 1u) == nsplit - 1 ? 1u : 0u;
      __syncthreads();
      if (last_s) {
        for (int g = wave; g < G; g += WAVES) {
          float L, n0, n1;
          merge_records<true>(part + ((uint64_t)r * qh + h * G + g) * smax * kAttnPartialFloats, nsplit, lane, L, n0,
                              n1);
          const uint32_t o0 = f32_to_bf16(n0 / L), o1 = f32_to_bf16(n1 / L);
          bad |= !(L > 0.f) | ((o0 & 0x7f80u) == 0x7f80u) | ((o1 & 0x7f80u) == 0x7f80u);
          store_head(out, out_mtiles, row0, r, qh, h * G + g, lane, o0, o1);
        }
        if (threadIdx.x == 0) atomicExch(counter, 0u);  // ready for the next launch
      }
    }
  }
  if (bad) raise_error(err, ERR_NONFINITE);
  if (bad_page) raise_error(err, ERR_PAGE);
}

__global__ __launch_bounds__(kAttnThreads) void attn_merge_kernel(const float* __restrict__ part,
                                                                  const uint32_t* __restrict__ positions,
                                                                  uint16_t* __restrict__ out, uint32_t out_mtiles,
                                                                  uint32_t row0, uint32_t rows, uint32_t qh,
                                                                  uint32_t context, uint32_t smax,
                                                                  uint32_t split_pages, uint32_t* err) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t id = blockIdx.x * 4 + wave;
  const uint32_t r = id / qh, head = id % qh;
  if (r >= rows) return;
  const uint32_t pos = positions[r];
  if (pos >= context) return;  // reported by the partition kernel
  const uint32_t row_pages = (pos + 16) / 16;
  const uint32_t ns = (row_pages + split_pages - 1) / split_pages;
  if (ns == 1) return;  // finished by the partition kernel
  float L, n0, n1;
  merge_records(part + ((uint64_t)r * qh + head) * smax * kAttnPartialFloats, ns, lane, L, n0, n1);
  const uint32_t o0 = f32_to_bf16(n0 / L), o1 = f32_to_bf16(n1 / L);
  store_head(out, out_mtiles, row0, r, qh, head, lane, o0, o1);
  if (!(L > 0.f) || ((o0 & 0x7f80u) == 0x7f80u) || ((o1 & 0x7f80u) == 0x7f80u)) raise_error(err, ERR_NONFINITE);
}

template <int G, int PP, bool FUSED, int QKS>
void launch_partition(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, const uint32_t* positions,
                      const uint32_t* table, float* part, uint16_t* out, uint32_t out_mtiles, uint32_t row0,
                      uint32_t rows, uint32_t qh, uint32_t kvh, uint32_t stride, uint32_t pages, uint32_t context,
                      uint32_t smax, uint32_t* counters, uint32_t* err, const AttnQkn& qk, hipStream_t s) {
  constexpr int kWaves = 8;
  hipLaunchKernelGGL((attn_partition_kernel<G, kWaves, PP, FUSED, QKS>), dim3(smax, kvh, rows), dim3(64 * kWaves), 0,
                     s, q, kc, vc, positions, table, part, out, out_mtiles, row0, qh, kvh, stride, pages, context, smax,
                     counters, err, qk);
}

template <int G, int PP, int QKS>
void launch_partition_pp(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, const uint32_t* positions,
                         const uint32_t* table, float* part, uint16_t* out, uint32_t out_mtiles, uint32_t row0,
                         uint32_t rows, uint32_t qh, uint32_t kvh, uint32_t stride, uint32_t pages, uint32_t context,
                         uint32_t smax, uint32_t* counters, uint32_t* err, const AttnQkn& qk, hipStream_t s) {
  if (counters)
    launch_partition<G, PP, true, QKS>(q, kc, vc, positions, table, part, out, out_mtiles, row0, rows, qh, kvh,
                                       stride, pages, context, smax, counters, err, qk, s);
  else
    launch_partition<G, PP, false, QKS>(q, kc, vc, positions, table, part, out, out_mtiles, row0, rows, qh, kvh,
                                        stride, pages, context, smax, counters, err, qk, s);
}

template <int G, int QKS>
hipError_t launch_partition_g(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, const uint32_t* positions,
                              const uint32_t* table, float* part, uint16_t* out, uint32_t out_mtiles, uint32_t row0,
                              uint32_t rows, uint32_t qh, uint32_t kvh, uint32_t stride, uint32_t pages,
                              uint32_t context, uint32_t split_pages, uint32_t* counters, uint32_t* err,
                              const AttnQkn& qk, hipStream_t s) {
  const uint32_t smax = attn_max_splits(context, split_pages);
  switch (split_pages) {
    case 16: launch_partition_pp<G, 16, QKS>(q, kc, vc, positions, table, part, out, out_mtiles, row0, rows, qh, kvh, stride, pages, context, smax, counters, err, qk, s); break;
    case 32: launch_partition_pp<G, 32, QKS>(q, kc, vc, positions, table, part, out, out_mtiles, row0, rows, qh, kvh, stride, pages, context, smax, counters, err, qk, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipSuccess;
}

}  // namespace

bool attention_qkn_supported(uint32_t qh, uint32_t kvh, uint32_t qkv_splits) {
  return kvh && qh % kvh == 0 && qh / kvh <= 4 && (qh / kvh & (qh / kvh - 1)) == 0 && qkv_splits == 2;
}

hipError_t launch_attention_partial(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                    const uint32_t* positions, const uint32_t* table, float* partials, uint16_t* out,
                                    uint32_t out_tiled, uint32_t row0, uint32_t out_rows, uint32_t rows, uint32_t qh,
                                    uint32_t kvh, uint32_t stride, uint32_t pages, uint32_t context,
                                    uint32_t split_pages, uint32_t* counters, uint32_t* err, hipStream_t s,
                                    const AttnQkn* qkn) {
  const uint32_t mt = out_tiled ? act_mtiles(out_rows) : 0u;
  hipError_t e;
  const AttnQkn none{};
  if (qkn) {
    if (!attention_qkn_supported(qh, kvh, qkn->splits) || row0 != 0) return hipErrorInvalidValue;
    switch (qh / kvh) {
      case 1: e = launch_partition_g<1, 2>(q, k_cache, v_cache, positions, table, partials, out, mt, row0, rows, qh, kvh, stride, pages, context, split_pages, counters, err, *qkn, s); break;
      case 2: e = launch_partition_g<2, 2>(q, k_cache, v_cache, positions, table, partials, out, mt, row0, rows, qh, kvh, stride, pages, context, split_pages, counters, err, *qkn, s); break;
      case 4: e = launch_partition_g<4, 2>(q, k_cache, v_cache, positions, table, partials, out, mt, row0, rows, qh, kvh, stride, pages, context, split_pages, counters, err, *qkn, s); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (qh / kvh) {
      case 1: e = launch_partition_g<1, 0>(q, k_cache, v_cache, positions, table, partials, out, mt, row0, rows, qh, kvh, stride, pages, context, split_pages, counters, err, none, s); break;
      case 2: e = launch_partition_g<2, 0>(q, k_cache, v_cache, positions, table, partials, out, mt, row0, rows, qh, kvh, stride, pages, context, split_pages, counters, err, none, s); break;
      case 4: e = launch_partition_g<4, 0>(q, k_cache, v_cache, positions, table, partials, out, mt, row0, rows, qh, kvh, stride, pages, context, split_pages, counters, err, none, s); break;
      case 8: e = launch_partition_g<8, 0>(q, k_cache, v_cache, positions, table, partials, out, mt, row0, rows, qh, kvh, stride, pages, context, split_pages, counters, err, none, s); break;
      default: return hipErrorInvalidValue;
    }
  }
  if (e != hipSuccess) return e;
  return hipGetLastError();
}

hipError_t launch_attention_merge(const float* partials, const uint32_t* positions, uint16_t* out,
                                  uint32_t out_tiled, uint32_t row0, uint32_t out_rows, uint32_t rows, uint32_t qh,
                                  uint32_t context, uint32_t split_pages, uint32_t* err, hipStream_t s) {
  if (split_pages != 16 && split_pages != 32) return hipErrorInvalidValue;
  const uint32_t smax = attn_max_splits(context, split_pages);
  const uint32_t waves = rows * qh;
  const uint32_t mt = out_tiled ? act_mtiles(out_rows) : 0u;
  hipLaunchKernelGGL(attn_merge_kernel, dim3((waves + 3) / 4), dim3(kAttnThreads), 0, s, partials, positions, out,
                     mt, row0, rows, qh, context, smax, split_pages, err);
  return hipGetLastError();
}

}  // namespace fh
