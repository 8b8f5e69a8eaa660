// Data-movement kernels: weight tiling, embedding gather, synthetic fills,
// KV prefix fill, small utilities. All HBM-bound byte work, one 16-byte
// chunk per lane where the layout allows.
#include "common.hpp"
#include "kernels.hpp"
#include "../../include/ferric_synth.h"

namespace fh {

namespace {

constexpr int kThreads = 256;

inline unsigned grid_for(uint64_t work, uint64_t per_block, unsigned cap = 1u << 20) {
  uint64_t g = (work + per_block - 1) / per_block;
  if (g == 0) g = 1;
  return (unsigned)(g < cap ? g : cap);
}

// One thread per 16-byte destination chunk. Source n-tile nt lands in
// destination n-tile nt * tile_mul + tile_add (tile_mul = 2 interleaves the
// gate and up projections tile by tile for the fused SwiGLU epilogue).
__global__ __launch_bounds__(kThreads) void tile_weight_kernel(const uint16_t* __restrict__ src,
                                                               uint16_t* __restrict__ dst, uint32_t n, uint32_t k,
                                                               uint32_t tile_mul, uint32_t tile_add) {
  const uint32_t kb_count = k >> 5;
  const uint64_t chunks = (uint64_t)n * k / 8;
  for (uint64_t c = (uint64_t)blockIdx.x * kThreads + threadIdx.x; c < chunks; c += (uint64_t)gridDim.x * kThreads) {
    uint64_t tile = c >> 6;
    uint32_t lane = (uint32_t)(c & 63u);
    uint64_t nb = tile / kb_count;
    uint32_t kb = (uint32_t)(tile - nb * kb_count);
    uint64_t row = nb * 16 + (lane & 15u);
    uint32_t col = kb * 32 + (lane >> 4) * 8;
    uint4 v = *reinterpret_cast<const uint4*>(src + row * k + col);
    uint64_t dtile = (nb * tile_mul + tile_add) * kb_count + kb;
    *reinterpret_cast<uint4*>(dst + ((dtile * 64 + lane) << 3)) = v;
  }
}

__global__ __launch_bounds__(kThreads) void untile_weight_kernel(const uint16_t* __restrict__ tiled,
                                                                 uint16_t* __restrict__ dst, uint32_t n, uint32_t k) {
  const uint32_t kb_count = k >> 5;
  const uint64_t chunks = (uint64_t)n * k / 8;
  for (uint64_t c = (uint64_t)blockIdx.x * kThreads + threadIdx.x; c < chunks; c += (uint64_t)gridDim.x * kThreads) {
    uint64_t tile = c >> 6;
    uint32_t lane = (uint32_t)(c & 63u);
    uint64_t nb = tile / kb_count;
    uint32_t kb = (uint32_t)(tile - nb * kb_count);
    uint64_t row = nb * 16 + (lane & 15u);
    uint32_t col = kb * 32 + (lane >> 4) * 8;
    *reinterpret_cast<uint4*>(dst + row * k + col) = *reinterpret_cast<const uint4*>(tiled + (c << 3));
  }
}

// Embedding gather straight out of the tiled table (one copy serves both the
// embedding and a tied LM head). Token ids >= vocab raise ERR_TOKEN and read
// row 0 instead of faulting (the reference traps:
// device/qwen3-all-kernels-v1/src/gemm.rs:768-853).
__global__ __launch_bounds__(kThreads) void embedding_kernel(const uint32_t* __restrict__ tokens,
                                                             const uint16_t* __restrict__ table,
                                                             uint16_t* __restrict__ out, uint32_t hidden,
                                                             uint32_t vocab, uint32_t* err) {
  const uint32_t row = blockIdx.x;
  uint32_t tok = tokens[row];
  if (tok >= vocab) {
    if (threadIdx.x == 0) raise_error(err, ERR_TOKEN);
    tok = 0;
  }
  const uint32_t kb_count = hidden >> 5;
  const uint32_t nb = tok >> 4, r = tok & 15u;
  for (uint32_t c = threadIdx.x; c < hidden / 8; c += kThreads) {
    uint32_t kb = c >> 2, g = c & 3u;
    uint64_t src = ((((uint64_t)nb * kb_count + kb) * 64u) + r + 16u * g) << 3;
    *reinterpret_cast<uint4*>(out + (uint64_t)row * hidden + c * 8) = *reinterpret_cast<const uint4*>(table + src);
  }
}

__global__ __launch_bounds__(kThreads) void synth_fill_kernel(uint16_t* __restrict__ dst, uint64_t count,
                                                              uint64_t tensor_seed, float scale) {
  // Eight samples per thread, stored as one 16-byte chunk where aligned.
  const uint64_t chunks = count / 8;
  for (uint64_t c = (uint64_t)blockIdx.x * kThreads + threadIdx.x; c < chunks; c += (uint64_t)gridDim.x * kThreads) {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t lo = fh_synth_bf16(tensor_seed, c * 8 + 2 * j, scale);
      uint32_t hi = fh_synth_bf16(tensor_seed, c * 8 + 2 * j + 1, scale);
      w[j] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(dst + c * 8) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  if (blockIdx.x == 0 && threadIdx.x < (count & 7u)) {
    uint64_t i = chunks * 8 + threadIdx.x;
    dst[i] = fh_synth_bf16(tensor_seed, i, scale);
  }
}

__global__ __launch_bounds__(kThreads) void fill_u16_kernel(uint16_t* __restrict__ dst, uint64_t count,
                                                            uint16_t value) {
  for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < count; i += (uint64_t)gridDim.x * kThreads)
    dst[i] = value;
}

// Synthetic KV prefix: blockIdx.y = row, blockIdx.x strides over
// (position, head, dim/8) chunks below lengths[row]. Values are keyed by the
// logical position, so any page permutation stores the same logical KV.
__global__ __launch_bounds__(kThreads) void kv_fill_kernel(uint16_t* __restrict__ cache,
                                                           const uint32_t* __restrict__ table,
                                                           const uint32_t* __restrict__ lengths,
                                                           const uint64_t* __restrict__ keys, uint32_t stride,
                                                           uint32_t kv_heads, uint64_t tensor_seed, float scale,
                                                           uint32_t context_stride) {
  const uint32_t row = blockIdx.y;
  const uint32_t len = lengths[row];
  const uint32_t row_elems = kv_heads * 128;
  const uint64_t chunks = (uint64_t)len * row_elems / 8;
  const uint64_t key = keys[row];
  for (uint64_t c = (uint64_t)blockIdx.x * kThreads + threadIdx.x; c < chunks; c += (uint64_t)gridDim.x * kThreads) {
    uint64_t e = c * 8;
    uint32_t pos = (uint32_t)(e / row_elems);
    uint32_t within = (uint32_t)(e - (uint64_t)pos * row_elems);
    uint32_t page = table[(uint64_t)row * stride + pos / 16];
    uint64_t dst = ((uint64_t)page * 16 + (pos & 15u)) * row_elems + within;
    uint64_t idx = ((key * context_stride) + pos) * row_elems + within;
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t lo = fh_synth_bf16(tensor_seed, idx + 2 * j, scale);
      uint32_t hi = fh_synth_bf16(tensor_seed, idx + 2 * j + 1, scale);
      w[j] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(cache + dst) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// dst[i][:] = src[index[i]][:] for i < rows (width % 8 == 0), one workgroup per row.
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(const uint16_t* __restrict__ src,
                                                               const uint32_t* __restrict__ index,
                                                               uint16_t* __restrict__ dst, uint32_t width) {
  const uint32_t row = blockIdx.x;
  const uint4* s = reinterpret_cast<const uint4*>(src + (uint64_t)index[row] * width);
  uint4* d = reinterpret_cast<uint4*>(dst + (uint64_t)row * width);
  for (uint32_t c = threadIdx.x; c < width / 8; c += kThreads) d[c] = s[c];
}

__global__ void clear_word_kernel(uint32_t* word) {
  if (threadIdx.x == 0) *word = 0u;
}

// System-scope loads read the coherent pinned buffer past every GPU cache, so
// each step sees what the host wrote before the launch.
// The first launch of a decode step. The metadata block (tokens, positions,
// page tables) comes in from coherent pinned host memory, one word per thread
// over the whole grid; workgroup r < rows also gathers row r's embedding, its
// token read once from the host block itself (the device copy is for the
// later launches). Workgroup 0 alone writes the step's error word: it clears
// it and raises ERR_TOKEN if any row's token is out of range (rows <= 64: one
// wave checks every row's token), so the word has one writer in this launch.
// Out-of-range tokens read row 0.
__global__ __launch_bounds__(kThreads) void step_embed_kernel(const uint32_t* __restrict__ host,
                                                              uint32_t* __restrict__ dev, uint32_t words,
                                                              const uint16_t* __restrict__ table,
                                                              uint16_t* __restrict__ out, uint32_t rows,
                                                              uint32_t hidden, uint32_t vocab, uint32_t* err) {
  __shared__ uint32_t tok_s;
  uint32_t* src = const_cast<uint32_t*>(host);
  const uint32_t blk = blockIdx.x;
  // The first word of this thread's share, this row's token and (wave 0 of
  // workgroup 0) the rows' tokens for the check are requested together: one
  // round trip over the host link instead of one after another.
  const uint32_t i0 = blk * kThreads + threadIdx.x;
  const uint32_t w0 = i0 < words ? __hip_atomic_load(src + i0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) : 0u;
  const uint32_t t0 =
      blk < rows && threadIdx.x == 0 ? __hip_atomic_load(src + blk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) : 0u;
  const uint32_t tc = blk == 0 && threadIdx.x < rows
                          ? __hip_atomic_load(src + threadIdx.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM)
                          : 0u;
  if (i0 < words) dev[i0] = w0;
  for (uint32_t i = i0 + gridDim.x * kThreads; i < words; i += gridDim.x * kThreads)
    dev[i] = __hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  if (blk == 0 && threadIdx.x < 64) {
    // Wave 0 of workgroup 0, lane r: row r's token.
    const bool any = __ballot(threadIdx.x < rows && tc >= vocab) != 0ull;
    if (threadIdx.x == 0 && err) *err = any ? (uint32_t)ERR_TOKEN : 0u;
  }
  if (blk >= rows) return;  // uniform per workgroup
  if (threadIdx.x == 0) tok_s = t0;
  __syncthreads();
  uint32_t tok = tok_s;
  if (tok >= vocab) tok = 0;
  const uint32_t kb_count = hidden >> 5;
  const uint32_t nb = tok >> 4, r = tok & 15u;
  for (uint32_t c = threadIdx.x; c < hidden / 8; c += kThreads) {
    uint32_t kb = c >> 2, g = c & 3u;
    uint64_t sidx = ((((uint64_t)nb * kb_count + kb) * 64u) + r + 16u * g) << 3;
    *reinterpret_cast<uint4*>(out + (uint64_t)blk * hidden + c * 8) = *reinterpret_cast<const uint4*>(table + sidx);
  }
}

__global__ __launch_bounds__(kThreads) void copy_u16_kernel(const uint16_t* __restrict__ src,
                                                            uint16_t* __restrict__ dst, uint64_t count) {
  const uint64_t chunks = count / 8;
  for (uint64_t c = (uint64_t)blockIdx.x * kThreads + threadIdx.x; c < chunks; c += (uint64_t)gridDim.x * kThreads)
    *reinterpret_cast<uint4*>(dst + c * 8) = *reinterpret_cast<const uint4*>(src + c * 8);
  if (blockIdx.x == 0 && threadIdx.x < (count & 7u)) dst[chunks * 8 + threadIdx.x] = src[chunks * 8 + threadIdx.x];
}

}  // namespace

hipError_t launch_tile_weight(const uint16_t* src, uint16_t* dst, uint32_t n, uint32_t k, uint32_t tile_mul,
                              uint32_t tile_add, hipStream_t s) {
  uint64_t chunks = (uint64_t)n * k / 8;
  hipLaunchKernelGGL(tile_weight_kernel, dim3(grid_for(chunks, kThreads, 65536)), dim3(kThreads), 0, s, src, dst, n,
                     k, tile_mul, tile_add);
  return hipGetLastError();
}

hipError_t launch_untile_weight(const uint16_t* tiled, uint16_t* dst, uint32_t n, uint32_t k, hipStream_t s) {
  uint64_t chunks = (uint64_t)n * k / 8;
  hipLaunchKernelGGL(untile_weight_kernel, dim3(grid_for(chunks, kThreads, 65536)), dim3(kThreads), 0, s, tiled, dst,
                     n, k);
  return hipGetLastError();
}

hipError_t launch_embedding(const uint32_t* tokens, const uint16_t* table_tiled, uint16_t* out, uint32_t rows,
                            uint32_t hidden, uint32_t vocab, uint32_t* err, hipStream_t s) {
  hipLaunchKernelGGL(embedding_kernel, dim3(rows), dim3(kThreads), 0, s, tokens, table_tiled, out, hidden, vocab, err);
  return hipGetLastError();
}

hipError_t launch_synth_fill(uint16_t* dst, uint64_t count, uint64_t tensor_seed, float scale, hipStream_t s) {
  hipLaunchKernelGGL(synth_fill_kernel, dim3(grid_for(count / 8 + 1, kThreads, 65536)), dim3(kThreads), 0, s, dst,
                     count, tensor_seed, scale);
  return hipGetLastError();
}

hipError_t launch_fill_u16(uint16_t* dst, uint64_t count, uint16_t value, hipStream_t s) {
  hipLaunchKernelGGL(fill_u16_kernel, dim3(grid_for(count, kThreads, 65536)), dim3(kThreads), 0, s, dst, count, value);
  return hipGetLastError();
}

hipError_t launch_kv_fill(uint16_t* cache, const uint32_t* table, const uint32_t* lengths, const uint64_t* keys,
                          uint32_t rows, uint32_t stride, uint32_t kv_heads, uint64_t tensor_seed, float scale,
                          uint32_t context_stride, uint32_t max_length, hipStream_t s) {
  uint64_t chunks = (uint64_t)max_length * kv_heads * 128 / 8;
  hipLaunchKernelGGL(kv_fill_kernel, dim3(grid_for(chunks, kThreads, 4096), rows), dim3(kThreads), 0, s, cache, table,
                     lengths, keys, stride, kv_heads, tensor_seed, scale, context_stride);
  return hipGetLastError();
}

hipError_t launch_gather_rows(const uint16_t* src, const uint32_t* index, uint16_t* dst, uint32_t rows,
                              uint32_t width, hipStream_t s) {
  hipLaunchKernelGGL(gather_rows_kernel, dim3(rows), dim3(kThreads), 0, s, src, index, dst, width);
  return hipGetLastError();
}

hipError_t launch_clear_word(uint32_t* word, hipStream_t s) {
  hipLaunchKernelGGL(clear_word_kernel, dim3(1), dim3(64), 0, s, word);
  return hipGetLastError();
}

hipError_t launch_step_embed(const uint32_t* host, uint32_t* dev, uint32_t words, const uint16_t* table_tiled,
                             uint16_t* out, uint32_t rows, uint32_t hidden, uint32_t vocab, uint32_t* err,
                             hipStream_t s) {
  if (rows == 0 || rows > 64 || words < rows) return hipErrorInvalidValue;
  const uint32_t grid = std::max<uint32_t>(rows, grid_for(words, kThreads, 256));
  hipLaunchKernelGGL(step_embed_kernel, dim3(grid), dim3(kThreads), 0, s, host, dev, words, table_tiled, out, rows,
                     hidden, vocab, err);
  return hipGetLastError();
}

hipError_t launch_copy_u16(const uint16_t* src, uint16_t* dst, uint64_t count, hipStream_t s) {
  hipLaunchKernelGGL(copy_u16_kernel, dim3(grid_for(count / 8 + 1, kThreads, 65536)), dim3(kThreads), 0, s, src, dst,
                     count);
  return hipGetLastError();
}

}  // namespace fh
