// K7 greedy choice: two-pass lowest-id argmax over FP32 logits.
//
// Reference rule (device/qwen3-all-kernels-v1/src/logits.rs:197-270 serial
// scan with strict '>', and the v11/v13 parallel forms,
// device/qwen3-tp-fp32-argmax-kernels-v11/src/logits.rs:58-153): the choice is
// the lowest token id whose logit equals the row maximum; any nonfinite logit
// in the row is an error. Pass 1 (grid rows x 64 shards) reduces one
// contiguous shard per workgroup; pass 2 (one wave per row) reduces the 64
// shard winners. Both passes break ties toward the lower id, so the result is
// the serial scan's, bit for bit, whatever the reduction tree.
#include "common.hpp"
#include "kernels.hpp"

namespace fh {

namespace {

constexpr int kArgThreads = 256;
constexpr uint32_t kNone = 0xffffffffu;

struct Cand {
  float v;
  uint32_t id;
};

__device__ __forceinline__ Cand better(Cand a, Cand b) {
  if (b.id == kNone) return a;
  if (a.id == kNone) return b;
  if (b.v > a.v || (b.v == a.v && b.id < a.id)) return b;
  return a;
}

__device__ __forceinline__ Cand wave_best(Cand c) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    Cand o{__shfl_xor(c.v, off, 64), (uint32_t)__shfl_xor((int)c.id, off, 64)};
    c = better(c, o);
  }
  return c;
}

__global__ __launch_bounds__(kArgThreads) void argmax_partial_kernel(const float* __restrict__ logits,
                                                                     uint32_t vocab, float* __restrict__ pval,
                                                                     uint32_t* __restrict__ pidx, uint32_t* err) {
  __shared__ Cand red[kArgThreads / 64];
  const uint32_t shard = blockIdx.x, row = blockIdx.y;
  const uint32_t chunk = (vocab + kArgmaxShards - 1) / kArgmaxShards;
  const uint32_t lo = shard * chunk;
  const uint32_t hi = min(lo + chunk, vocab);
  const float* lr = logits + (uint64_t)row * vocab;
  Cand best{0.f, kNone};
  bool bad = false;
  for (uint32_t i = lo + threadIdx.x; i < hi; i += kArgThreads) {
    const float v = lr[i];
    if (!is_finite_f32(v)) {
      bad = true;
    } else if (best.id == kNone || v > best.v) {
      best.v = v;
      best.id = i;
    }
  }
  best = wave_best(best);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    Cand c = red[0];
#pragma unroll
    for (int w = 1; w < kArgThreads / 64; ++w) c = better(c, red[w]);
    pval[row * kArgmaxShards + shard] = c.v;
    pidx[row * kArgmaxShards + shard] = c.id;
  }
  if (bad) raise_error(err, ERR_NONFINITE);
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const float* __restrict__ pval,
                                                          const uint32_t* __restrict__ pidx,
                                                          uint32_t* __restrict__ choices, uint32_t* err,
                                                          uint32_t* host_choices, uint32_t* host_err,
                                                          uint32_t* host_done) {
  const uint32_t row = blockIdx.x;
  Cand c{pval[row * kArgmaxShards + threadIdx.x], pidx[row * kArgmaxShards + threadIdx.x]};
  c = wave_best(c);
  if (threadIdx.x == 0) {
    const uint32_t id = c.id == kNone ? 0u : c.id;
    choices[row] = id;
    if (c.id == kNone) raise_error(err, ERR_NONFINITE);
    if (host_choices) {
      __hip_atomic_store(host_choices + row, id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      if (row == 0) {
        // Every earlier launch has completed, and a row with no finite logit
        // raised ERR_NONFINITE in the partial pass already, so the word read
        // here holds every error bit the step can report.
        const uint32_t e = err ? __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
        __hip_atomic_store(host_err, e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      }
      // Published after this row's stores above: a host that sees the word
      // set reads this row's choice (and, for row 0, the error word).
      if (host_done) __hip_atomic_store(host_done + row, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
}

}  // namespace

hipError_t launch_argmax(const float* logits, uint32_t rows, uint32_t vocab, void* scratch, uint32_t* choices,
                         uint32_t* err, hipStream_t s, uint32_t* host_choices, uint32_t* host_err,
                         uint32_t* host_done) {
  float* pval = reinterpret_cast<float*>(scratch);
  uint32_t* pidx = reinterpret_cast<uint32_t*>(pval + (uint64_t)rows * kArgmaxShards);
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgmaxShards, rows), dim3(kArgThreads), 0, s, logits, vocab, pval,
                     pidx, err);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(argmax_final_kernel, dim3(rows), dim3(64), 0, s, pval, pidx, choices, err,
                     host_choices, host_err, host_done);
  return hipGetLastError();
}

}  // namespace fh
