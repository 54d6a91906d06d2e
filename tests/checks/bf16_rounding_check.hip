// Exhaustive check of the FP32 -> BF16 conversion every kernel of this
// library uses for its BF16 outputs (loom_dev::bf16x2_pack, gfx950's
// v_cvt_pk_bf16_f32) against the integer form of half::bf16::from_f32:
// round to nearest even, and a NaN keeps its sign and top payload bits with
// the quiet bit set.  Every one of the 2^32 FP32 bit patterns is converted in
// both halves of the packed pair.  Prints the mismatch count; exit status 0
// only when it is zero.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

#include "attn_device.hpp"

namespace {

__device__ __forceinline__ uint32_t bf16_bits_reference(float f) {
  uint32_t x = __float_as_uint(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (x >> 16) | 0x40u;
  x += 0x7fffu + ((x >> 16) & 1u);
  return x >> 16;
}

// Launch `part` covers the 2^30 patterns (part << 30) + [0, 2^30): 2^26
// threads of 16 patterns each, in pairs (x, x + 1).
__global__ void check_kernel(uint32_t part, unsigned long long *mismatches, uint32_t *first) {
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  unsigned long long local = 0;
  for (int j = 0; j < 16; j += 2) {
    const uint32_t x0 = (uint32_t)(((uint64_t)part << 30) + t * 16 + (uint64_t)j);
    const float a = __uint_as_float(x0), b = __uint_as_float(x0 + 1u);
    const uint32_t ra = bf16_bits_reference(a), rb = bf16_bits_reference(b);
    const bool bad = loom_dev::bf16x2_pack(a, b) != (ra | (rb << 16)) ||
                     loom_dev::bf16x2_pack(b, a) != (rb | (ra << 16));
    if (bad) {
      ++local;
      atomicMin(first, x0);
    }
  }
  if (local) atomicAdd(mismatches, local);
}

}  // namespace

int main() {
  unsigned long long *mismatches = nullptr;
  uint32_t *first = nullptr;
  if (hipMalloc(&mismatches, sizeof(unsigned long long)) != hipSuccess ||
      hipMalloc(&first, sizeof(uint32_t)) != hipSuccess) {
    std::fprintf(stderr, "hipMalloc failed\n");
    return 2;
  }
  const uint32_t none = 0xffffffffu;
  if (hipMemset(mismatches, 0, sizeof(unsigned long long)) != hipSuccess ||
      hipMemcpy(first, &none, sizeof(none), hipMemcpyHostToDevice) != hipSuccess) {
    std::fprintf(stderr, "initialisation failed\n");
    return 2;
  }
  for (uint32_t part = 0; part < 4; ++part)
    hipLaunchKernelGGL(check_kernel, dim3(1u << 18), dim3(256), 0, 0, part, mismatches, first);
  unsigned long long count = 0;
  uint32_t first_bad = 0;
  if (hipDeviceSynchronize() != hipSuccess ||
      hipMemcpy(&count, mismatches, sizeof(count), hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(&first_bad, first, sizeof(first_bad), hipMemcpyDeviceToHost) != hipSuccess) {
    std::fprintf(stderr, "check failed: %s\n", hipGetErrorString(hipGetLastError()));
    return 2;
  }
  std::printf("bf16 rounding: 4294967296 patterns, %llu mismatching pairs", count);
  if (count) std::printf(", first at 0x%08x", first_bad);
  std::printf("\n");
  hipFree(mismatches);
  hipFree(first);
  return count == 0 ? 0 : 1;
}
