/*
 * ferric_synth.h — the synthetic-input convention shared by the HIP library
 * (which generates weights and KV prefixes directly in HBM) and the CPU
 * oracle (which regenerates the same bits on the host).
 *
 * The reference has no synthetic-weight generator of its own: its model-level
 * checks use the real Qwen3 checkpoint. The configurations this library is
 * measured on ask for "random-init bf16 weights ~N(0, sigma), norms = 1" and
 * "random KV bf16 ~N(0,1)". This header fixes one bit-exact definition of
 * that so both sides agree without shipping gigabytes of weights:
 *
 *   h      = splitmix64(tensor_seed + index)
 *   s      = sum of the four 16-bit fields of h            (integer, exact)
 *   z      = (float)(s - 131070) * scale                   (one IEEE f32 multiply)
 *   value  = bf16_rne(z)
 *
 * s is the Irwin-Hall sum of four uniform 16-bit integers: mean 131070,
 * standard deviation 65536/sqrt(3) = 37837.23. With
 * scale = sigma / 37837.23 (computed in double, rounded once to f32) the
 * value is an approximately normal N(0, sigma) sample bounded to +-3.46 sigma.
 * Every step is integer arithmetic or a single correctly rounded f32
 * multiply, so a CPU and a gfx950 kernel produce identical bits.
 *
 * Per-tensor seeds: tensor_seed = splitmix64(seed ^ splitmix64(kind * 2^32 + layer + 1)).
 * KV prefixes use kind = 100 (K) / 101 (V) and an element index of
 * (((sequence_key * context_stride + position) * kv_heads + head) * head_dim + dim),
 * so the values depend on the logical position only, never on which
 * physical page holds them.
 */
#ifndef FERRIC_SYNTH_H
#define FERRIC_SYNTH_H

#include <stdint.h>

#if defined(__HIPCC__)
#define FH_SYNTH_FN static inline __host__ __device__
#else
#define FH_SYNTH_FN static inline
#endif

#define FH_SYNTH_IRWIN_HALL_MEAN 131070
#define FH_SYNTH_IRWIN_HALL_STD 37837.2306413553 /* 65536 / sqrt(3) */
#define FH_SYNTH_KIND_KV_KEY 100u
#define FH_SYNTH_KIND_KV_VALUE 101u

FH_SYNTH_FN uint64_t fh_splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  uint64_t z = x;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

FH_SYNTH_FN uint64_t fh_synth_tensor_seed(uint64_t seed, uint32_t kind, uint32_t layer) {
  return fh_splitmix64(seed ^ fh_splitmix64(((uint64_t)kind << 32) + (uint64_t)layer + 1ull));
}

/* Integer part of one sample: s - mean, in [-131070, 131070]. */
FH_SYNTH_FN int32_t fh_synth_centered(uint64_t tensor_seed, uint64_t index) {
  uint64_t h = fh_splitmix64(tensor_seed + index);
  int32_t s = (int32_t)(h & 0xffffu) + (int32_t)((h >> 16) & 0xffffu) +
              (int32_t)((h >> 32) & 0xffffu) + (int32_t)((h >> 48) & 0xffffu);
  return s - FH_SYNTH_IRWIN_HALL_MEAN;
}

/* f32 scale for a target standard deviation; computed once on the host. */
static inline float fh_synth_scale(double sigma) {
  return (float)(sigma / FH_SYNTH_IRWIN_HALL_STD);
}

/* bf16 round-to-nearest-even with quiet-NaN marking (see the library's
 * bf16 helpers for the citation of the reference rule). */
FH_SYNTH_FN uint16_t fh_synth_bf16_rne(float value) {
  union {
    float f;
    uint32_t u;
  } bits;
  bits.f = value;
  uint32_t b = bits.u;
  if ((b & 0x7f800000u) == 0x7f800000u && (b & 0x007fffffu) != 0u) {
    return (uint16_t)((b >> 16) | 0x0040u);
  }
  return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

FH_SYNTH_FN uint16_t fh_synth_bf16(uint64_t tensor_seed, uint64_t index, float scale) {
  return fh_synth_bf16_rne((float)fh_synth_centered(tensor_seed, index) * scale);
}

#endif /* FERRIC_SYNTH_H */
