// bench_read.hip -- measurement aid for bench.py (libullm_bench.so): a plain
// streaming read of a device buffer, the floor a kernel that must read every
// byte of a weight matrix once cannot beat at that size.
//
// Each wave reads a contiguous 16 KiB run of the buffer (16 independent
// 1 KiB dwordx4 loads in flight per wave), XOR-folds it and writes one word
// per workgroup, so no load can be optimised away.  One workgroup of 8 waves
// covers 128 KiB; the grid covers the buffer.  Not part of the quantized
// linear layer: it computes nothing the layer needs.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr uint32_t kWaves = 8;
constexpr uint32_t kLoads = 16;  // 1 KiB per wave per load
constexpr uint64_t kWaveBytes = kLoads * 1024;
constexpr uint64_t kBlockBytes = kWaves * kWaveBytes;

__global__ __launch_bounds__(kWaves * 64) void stream_read_kernel(
    const u32x4 *__restrict__ src, uint64_t vecs, uint32_t *__restrict__ sink) {
  const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const uint64_t base = (uint64_t(blockIdx.x) * kBlockBytes + wave * kWaveBytes) / 16;
  u32x4 acc = {0u, 0u, 0u, 0u};
  u32x4 v[kLoads];
#pragma unroll
  for (uint32_t i = 0; i < kLoads; ++i) {
    const uint64_t idx = base + i * 64 + lane;
    v[i] = idx < vecs ? src[idx] : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (uint32_t i = 0; i < kLoads; ++i) {
    acc ^= v[i];
  }
  uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
  for (int off = 32; off > 0; off >>= 1) {
    r ^= __shfl_xor(r, off);
  }
  __shared__ uint32_t part[kWaves];
  if (lane == 0) part[wave] = r;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
    for (uint32_t w = 0; w < kWaves; ++w) t ^= part[w];
    sink[blockIdx.x] = t;
  }
}

}  // namespace

// Reads `bytes` (a multiple of 16) at `src`; `sink` holds one u32 per
// 128 KiB of input.  Returns the launch status.
extern "C" __attribute__((visibility("default"))) int ullm_bench_stream_read(
    const void *src, uint64_t bytes, uint32_t *sink, void *stream) {
  const uint64_t blocks = (bytes + kBlockBytes - 1) / kBlockBytes;
  hipLaunchKernelGGL(stream_read_kernel, dim3(uint32_t(blocks)), dim3(kWaves * 64), 0,
                     static_cast<hipStream_t>(stream),
                     static_cast<const u32x4 *>(src), bytes / 16, sink);
  return int(hipGetLastError());
}
