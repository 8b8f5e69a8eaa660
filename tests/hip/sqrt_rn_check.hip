// Exhaustive check of the device's correctly rounded square root (sqrt_rn in
// ferric_amd/csrc/qk_head.hpp, the root inside every RMSNorm): for every
// positive normal float x, r = sqrt_rn(x) must lie in the rounding interval
// of sqrt(x), i.e. m_lo^2 < x < m_hi^2 with m_lo, m_hi the midpoints between
// r and its neighbouring floats. The midpoints carry at most 25 significant
// bits, so their squares are exact in double precision and the comparison is
// exact (a float's root never lies on a midpoint). Prints the count of
// inputs checked and of failures (with the first failing input); exits 1 on
// any failure.
#include <cstdio>
#include <cstdint>

#include "../../ferric_amd/csrc/qk_head.hpp"

namespace {

constexpr uint32_t kFirst = 0x00800000u;  // smallest positive normal
constexpr uint32_t kLast = 0x7f7fffffu;   // largest finite

__global__ void check_kernel(unsigned long long* failures, uint32_t* first_bad, uint32_t* last_bad) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  unsigned long long bad = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i <= kLast - kFirst; i += stride) {
    const uint32_t bits = kFirst + (uint32_t)i;
    const float x = __builtin_bit_cast(float, bits);
    const float r = fh::sqrt_rn(x);
    const uint32_t rb = __builtin_bit_cast(uint32_t, r);
    const double rd = (double)r;
    const double lo = (rd + (double)__builtin_bit_cast(float, rb - 1u)) * 0.5;
    const double hi = (rd + (double)__builtin_bit_cast(float, rb + 1u)) * 0.5;
    const double xd = (double)x;
    if (!(lo * lo < xd && xd < hi * hi)) {
      ++bad;
      atomicMin(first_bad, bits);
      atomicMax(last_bad, bits);
    }
  }
  if (bad) atomicAdd(failures, bad);
}

}  // namespace

int main() {
  unsigned long long* failures = nullptr;
  uint32_t* first_bad = nullptr;
  uint32_t* last_bad = nullptr;
  if (hipMalloc(&failures, sizeof(*failures)) != hipSuccess || hipMalloc(&first_bad, sizeof(*first_bad)) != hipSuccess ||
      hipMalloc(&last_bad, sizeof(*last_bad)) != hipSuccess) {
    fprintf(stderr, "hipMalloc failed\n");
    return 2;
  }
  hipMemset(failures, 0, sizeof(*failures));
  hipMemset(first_bad, 0xff, sizeof(*first_bad));
  hipMemset(last_bad, 0, sizeof(*last_bad));
  hipLaunchKernelGGL(check_kernel, dim3(16384), dim3(256), 0, 0, failures, first_bad, last_bad);
  unsigned long long f = 0;
  uint32_t fb = 0, lb = 0;
  if (hipDeviceSynchronize() != hipSuccess || hipMemcpy(&f, failures, sizeof(f), hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(&fb, first_bad, sizeof(fb), hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(&lb, last_bad, sizeof(lb), hipMemcpyDeviceToHost) != hipSuccess) {
    fprintf(stderr, "device error\n");
    return 2;
  }
  printf("checked %u positive normal floats, failures %llu", kLast - kFirst + 1, f);
  if (f) printf(", failing inputs from 0x%08x to 0x%08x", fb, lb);
  printf("\n");
  hipFree(failures);
  hipFree(first_bad);
  hipFree(last_bad);
  return f ? 1 : 0;
}
