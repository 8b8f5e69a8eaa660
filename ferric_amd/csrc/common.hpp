// Shared device helpers for the gfx950 kernels: bf16 carriers, wave64
// reductions, MFMA operand types and the error word.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fh {

// ---- bf16 carriers -------------------------------------------------------
// Narrowing is round-to-nearest-even on the f32 bit pattern; NaN payloads are
// quieted by setting bit 6 of the bf16 (0x0040). This is the rule the
// reference pins in device/qwen3-gemm-v1/tests/reference.rs:3-11 and :112-135
// (e.g. 0x3f808000 -> 0x3f80, 0x3f818000 -> 0x3f82, 0x7fa10001 -> 0x7fe1).

__host__ __device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __builtin_bit_cast(float, bits16 << 16);
}

// The narrowing as integer operations on the bit pattern.
__host__ __device__ __forceinline__ uint32_t f32_to_bf16_int(float v) {
  uint32_t b = __builtin_bit_cast(uint32_t, v);
  if ((b & 0x7f800000u) == 0x7f800000u && (b & 0x007fffffu) != 0u) return ((b >> 16) | 0x0040u) & 0xffffu;
  return (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
}

// On the device this is gfx950's v_cvt_pk_bf16_f32 (what a __bf16 cast
// compiles to): one instruction instead of the integer sequence, and equal to
// it for all 2^32 inputs, NaN payloads included (compared exhaustively on an
// MI355X).
__host__ __device__ __forceinline__ uint32_t f32_to_bf16(float v) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(uint16_t, (__bf16)v);
#else
  return f32_to_bf16_int(v);
#endif
}

// Two narrowings packed into one dword (lo in bits 0-15): one instruction on
// the device.
__host__ __device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
#if defined(__HIP_DEVICE_COMPILE__)
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
#else
  return f32_to_bf16(lo) | (f32_to_bf16(hi) << 16);
#endif
}

// Value after a round trip through bf16 (the reference's intermediate narrowing).
__device__ __forceinline__ float round_bf16(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__device__ __forceinline__ bool is_finite_f32(float v) {
  return (__builtin_bit_cast(uint32_t, v) & 0x7f800000u) != 0x7f800000u;
}

// Low / high bf16 of a packed dword, widened.
__device__ __forceinline__ float lo_bf16(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

// ---- error word -----------------------------------------------------------
// Kernels never trap: where the reference traps (nonfinite value, index out of
// range) they OR a bit into a device word that the host checks after the step.
enum : uint32_t {
  ERR_NONFINITE = 1u,
  ERR_TOKEN = 2u,
  ERR_POSITION = 4u,
  ERR_PAGE = 8u,
};

__device__ __forceinline__ void raise_error(uint32_t* err, uint32_t bit) {
  if (err) atomicOr(err, bit);
}

// ---- wave64 reductions (fixed butterfly order: deterministic) -------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Value of lane src (a wave-uniform index), read into every lane.
__device__ __forceinline__ float lane_bcast(float v, int src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), src));
}

// ---- MFMA operand types (gfx950 v_mfma_f32_16x16x32_bf16) -----------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// Tile order of a projection weight W[n][k] (n % 16 == 0, k % 32 == 0): a
// 16-row x 32-column tile is 1 KiB, stored as 64 lanes x 16 bytes in the exact
// order the MFMA A operand wants it (lane = row + 16 * (col / 8), 8 bf16 per
// lane). Tiles are stored tile-row major: tile (nb, kb) at (nb * KB + kb) KiB.
__host__ __device__ __forceinline__ uint64_t tiled_offset(uint32_t n, uint32_t k, uint32_t K) {
  uint32_t kb_count = K >> 5;
  uint32_t nb = n >> 4, r = n & 15u, kb = k >> 5, kk = k & 31u;
  uint32_t lane = r + 16u * (kk >> 3);
  return ((((uint64_t)nb * kb_count + kb) * 64u + lane) << 3) + (kk & 7u);
}

// Activation tile order: the B operand of the same MFMA for an activation
// x[m][k]. Tile (kb, mt) holds rows 16*mt..16*mt+15 and columns
// 32*kb..32*kb+31 as 64 lanes x 16 bytes (lane = m % 16 + 16 * ((k % 32) / 8));
// tiles are ordered kb-major over `mtiles` row tiles, so a wave's B-operand
// load is one contiguous 1 KiB. Producers of projection inputs (RMSNorm, the
// attention output, the SwiGLU epilogue) write this order directly. Decode
// buffers hold 32 rows (mtiles = 2); prefill buffers hold mtiles row tiles.
__host__ __device__ __forceinline__ uint64_t act_offset_m(uint32_t m, uint32_t k, uint32_t mtiles) {
  const uint32_t kb = k >> 5, kk = k & 31u, mt = m >> 4;
  const uint32_t lane = (m & 15u) + 16u * (kk >> 3);
  return ((((uint64_t)kb * mtiles + mt) * 64u + lane) << 3) + (kk & 7u);
}
__host__ __device__ __forceinline__ uint64_t act_offset(uint32_t m, uint32_t k) { return act_offset_m(m, k, 2); }

// SwiGLU element in the stable-sigmoid form of qwen3_swiglu_element_v1
// (device/qwen3-all-kernels-v1/src/swiglu.rs:62-101): e = exp(-|g|),
// sigmoid = (g >= 0 ? 1 : e) / (1 + e), y = bf16((g * sigmoid) * u).
__device__ __forceinline__ uint32_t swiglu_bf16(float g, float u, bool& bad) {
  bool nonneg = g >= 0.0f;
  float e = expf(nonneg ? -g : g);
  float denom = 1.0f + e;
  float sig = __fdiv_rn(nonneg ? 1.0f : e, denom);
  float silu = g * sig;
  float prod = silu * u;
  uint32_t out = f32_to_bf16(prod);
  bad |= !is_finite_f32(g) | !is_finite_f32(u) | ((out & 0x7f80u) == 0x7f80u);
  return out;
}

}  // namespace fh
