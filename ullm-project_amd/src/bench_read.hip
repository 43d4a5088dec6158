// bench_read.hip -- measurement aid for bench.py (libullm_bench.so): plain
// streaming reads of a device buffer, the floor that a kernel which must read
// every byte of a weight matrix once cannot beat at that size.
//
// stream_read_kernel<W, D>: workgroups of W waves; each wave streams its own
// contiguous `chunk` bytes as rounds of D independent 1 KiB loads (16 bytes
// per lane, non-temporal), XOR-folds them and writes one word per wave only
// when the fold hits a sentinel, so no load can be optimised away.  bench.py
// times a few (W, D, chunk) shapes and reports the fastest: on MI355X the
// best at 9-62 MB were 4 waves with 4-8 loads in flight over 4-8 KiB per
// wave.  Not part of the quantized linear layer.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {

template <int W, int D>
__global__ __launch_bounds__(W * 64) void stream_read_kernel(
    const u32x4 *__restrict__ src, uint64_t vecs, uint32_t chunk_vecs,
    uint32_t *__restrict__ sink) {
  const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const uint64_t base = (uint64_t(blockIdx.x) * W + wave) * chunk_vecs;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (uint32_t o = 0; o < chunk_vecs; o += D * 64) {
    u32x4 v[D];
#pragma unroll
    for (int i = 0; i < D; ++i) {
      const uint64_t idx = base + o + i * 64 + lane;
      v[i] = idx < vecs ? __builtin_nontemporal_load(src + idx) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < D; ++i) {
      acc ^= v[i];
    }
  }
  const uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (r == 0x9e3779b9u) {
    sink[blockIdx.x * W + wave] = r;
  }
}

template <int W, int D>
int launch(const void *src, uint64_t bytes, uint32_t chunk, uint32_t *sink,
           hipStream_t s) {
  const uint64_t vecs = bytes / 16, cv = chunk / 16;
  const uint64_t waves = (vecs + cv - 1) / cv;
  const uint32_t blocks = uint32_t((waves + W - 1) / W);
  hipLaunchKernelGGL((stream_read_kernel<W, D>), dim3(blocks), dim3(W * 64), 0, s,
                     static_cast<const u32x4 *>(src), vecs, uint32_t(cv), sink);
  return int(hipGetLastError());
}

}  // namespace

// Shape `shape` (0: 4 waves x 4 loads over 4 KiB per wave; 1: 4 x 8 over
// 8 KiB; 2: 8 x 8 over 8 KiB) reads `bytes` (a multiple of 16) at `src`;
// `sink` must hold one u32 per 1 KiB of input.  Returns the launch status.
extern "C" __attribute__((visibility("default"))) int ullm_bench_stream_read(
    const void *src, uint64_t bytes, uint32_t shape, uint32_t *sink, void *stream) {
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (shape) {
    case 0: return launch<4, 4>(src, bytes, 4096, sink, s);
    case 1: return launch<4, 8>(src, bytes, 8192, sink, s);
    default: return launch<8, 8>(src, bytes, 8192, sink, s);
  }
}

// The sweep of read shapes behind the floor: `waves` per workgroup (1, 2, 4,
// 8 or 16), `depth` independent 1 KiB loads in flight per wave (1, 2, 4, 8,
// 16 or 32), `chunk` bytes per wave (a multiple of depth x 1 KiB),
// non-temporal loads.  Returns hipErrorInvalidValue for any other shape.
template <int W>
int launch_depth(const void *src, uint64_t bytes, uint32_t depth, uint32_t chunk,
                 uint32_t *sink, hipStream_t s) {
  switch (depth) {
    case 1: return launch<W, 1>(src, bytes, chunk, sink, s);
    case 2: return launch<W, 2>(src, bytes, chunk, sink, s);
    case 4: return launch<W, 4>(src, bytes, chunk, sink, s);
    case 8: return launch<W, 8>(src, bytes, chunk, sink, s);
    case 16: return launch<W, 16>(src, bytes, chunk, sink, s);
    case 32: return launch<W, 32>(src, bytes, chunk, sink, s);
    default: return int(hipErrorInvalidValue);
  }
}

extern "C" __attribute__((visibility("default"))) int ullm_bench_stream_read_shape(
    const void *src, uint64_t bytes, uint32_t waves, uint32_t depth, uint32_t chunk,
    uint32_t *sink, void *stream) {
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (chunk == 0 || chunk % (depth * 1024u) != 0) {
    return int(hipErrorInvalidValue);
  }
  switch (waves) {
    case 1: return launch_depth<1>(src, bytes, depth, chunk, sink, s);
    case 2: return launch_depth<2>(src, bytes, depth, chunk, sink, s);
    case 4: return launch_depth<4>(src, bytes, depth, chunk, sink, s);
    case 8: return launch_depth<8>(src, bytes, depth, chunk, sink, s);
    case 16: return launch_depth<16>(src, bytes, depth, chunk, sink, s);
    default: return int(hipErrorInvalidValue);
  }
}
