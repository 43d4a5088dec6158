// check_bf16.hip -- test aid (libullm_bench.so, not part of the quantized
// linear layer): re-checks on a device that the f32 -> bf16 encode the
// kernels use (device_common.hpp: f32_to_bf16, f32x2_to_bf16x2, both the
// hardware convert) equals round-to-nearest-even on the 16 dropped bits with
// NaN kept quiet, over every one of the 2^32 f32 bit patterns.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device_common.hpp"

namespace {

// The rule, spelled out in integer arithmetic.
__device__ __forceinline__ uint16_t rne_rule(uint32_t b) {
  if ((b & 0x7fffffffu) > 0x7f800000u) {
    return static_cast<uint16_t>((b >> 16) | 0x0040u);
  }
  return static_cast<uint16_t>((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

// Each thread checks the pair (2 i, 2 i + 1) of its chunk through both the
// scalar and the packed encode.  counts: [0] finite or infinite mismatches,
// [1] NaN mismatches, [2] first mismatching input + 1 (0: none).
__global__ __launch_bounds__(256) void bf16_check_kernel(uint32_t base,
                                                         unsigned long long *counts) {
  const uint32_t i = base + 2u * (blockIdx.x * 256u + threadIdx.x);
  const uint32_t b0 = i, b1 = i + 1u;
  const float x0 = __builtin_bit_cast(float, b0), x1 = __builtin_bit_cast(float, b1);
  const uint32_t want = uint32_t(rne_rule(b0)) | (uint32_t(rne_rule(b1)) << 16);
  const uint32_t scalar = uint32_t(ullm::f32_to_bf16(x0)) |
                          (uint32_t(ullm::f32_to_bf16(x1)) << 16);
  const uint32_t packed = ullm::f32x2_to_bf16x2(x0, x1);
  if (scalar != want || packed != want) {
    const bool nan = (b0 & 0x7fffffffu) > 0x7f800000u || (b1 & 0x7fffffffu) > 0x7f800000u;
    atomicAdd(&counts[nan ? 1 : 0], 1ull);
    atomicCAS(&counts[2], 0ull, static_cast<unsigned long long>(b0) + 1ull);
  }
}

}  // namespace

// Checks all 2^32 inputs on `stream`; `counts` (3 device u64, zeroed by the
// caller) receives the mismatch counts.  Returns the launch status.
extern "C" __attribute__((visibility("default"))) int ullm_bench_bf16_convert_check(
    unsigned long long *counts, void *stream) {
  const hipStream_t s = static_cast<hipStream_t>(stream);
  constexpr uint64_t kPerLaunch = uint64_t(1) << 28;  // inputs per launch
  for (uint64_t base = 0; base < (uint64_t(1) << 32); base += kPerLaunch) {
    hipLaunchKernelGGL(bf16_check_kernel, dim3(uint32_t(kPerLaunch / 512)), dim3(256), 0, s,
                       uint32_t(base), counts);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
      return int(e);
    }
  }
  return 0;
}
