// gemm_fp8.hip -- prefill FP8 x FP8 GEMM on the gfx950 matrix cores.
//
// Y[m, n] = alpha * ((a_m * s_n) * sum_k e4m3(XA[m, k]) * e4m3(Q[n, k])),
// XA row-major [M][ldxq] (per-token scales a_m), Q in the FP8 wave-tile
// layout of layout.hpp (per-row scales s_n), fp32 accumulation.
//
// Direct-from-L2 version: every wave loads its operands straight from global
// memory in MFMA lane order (the weight tiles already are), with no LDS
// staging.  Correct for every shape; the LDS-pipelined kernel replaces it on
// the hot shapes.
#include "device_common.hpp"
#include "kernels.hpp"

#include "weight.hpp"

namespace ullm {
namespace {

typedef long i64;

__device__ __forceinline__ f32x4 mfma_fp8(i64 a, i64 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(a, b, c, 0, 0, 0);
}

// 16 activation bytes of row m at k0 (zero beyond M or K).
__device__ __forceinline__ u32x4 load_xq16(const uint8_t *__restrict__ row,
                                           bool valid, uint32_t k0, uint32_t K,
                                           bool vec) {
  u32x4 r = {0u, 0u, 0u, 0u};
  if (valid) {
    if (vec && k0 + 16 <= K) {
      r = *reinterpret_cast<const u32x4 *>(row + k0);
    } else {
      uint32_t b[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t v = (k0 + i < K) ? row[k0 + i] : 0u;
        b[i / 4] |= v << (8 * (i % 4));
      }
      r = u32x4{b[0], b[1], b[2], b[3]};
    }
  }
  return r;
}

struct GemmArgs {
  const uint8_t *xq;
  const float *xs;
  const uint8_t *tiles;
  const float *scales;
  void *y;
  uint64_t ldxq, ldy;
  uint32_t m, n, k, units;
  float alpha;
  bool y_f32;
};

// 256 threads, block tile 64 (m) x 64 (n); wave (wm, wn) owns 32 x 32.
__global__ __launch_bounds__(256) void fp8_gemm_direct_kernel(GemmArgs a,
                                                              bool vec) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const uint32_t m0 = blockIdx.y * 64 + (wave / 2) * 32;
  const uint32_t T0 = blockIdx.x * 4 + (wave % 2) * 2;  // 16-row stripes
  const uint32_t stripes = (a.n + 15) / 16;
  const uint8_t *rows[2];
  bool valid[2];
  for (int i = 0; i < 2; ++i) {
    const uint32_t m = m0 + i * 16 + lane % 16;
    valid[i] = m < a.m;
    rows[i] = a.xq + uint64_t(valid[i] ? m : 0) * a.ldxq;
  }
  f32x4 acc[2][2];
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const uint32_t kl = 16 * (lane / 16);
  for (uint32_t u = 0; u < a.units; ++u) {
    u32x4 bw[2];
    for (int j = 0; j < 2; ++j) {
      const uint32_t T = T0 + j < stripes ? T0 + j : stripes - 1;
      bw[j] = *reinterpret_cast<const u32x4 *>(
          a.tiles + (uint64_t(T) * a.units + u) * 1024 + lane * 16);
    }
    for (int i = 0; i < 2; ++i) {
      const u32x4 av = load_xq16(rows[i], valid[i], u * 64 + kl, a.k, vec);
      const i64 a0 = __builtin_bit_cast(i64, u32x2{av.x, av.y});
      const i64 a1 = __builtin_bit_cast(i64, u32x2{av.z, av.w});
      for (int j = 0; j < 2; ++j) {
        const i64 b0 = __builtin_bit_cast(i64, u32x2{bw[j].x, bw[j].y});
        const i64 b1 = __builtin_bit_cast(i64, u32x2{bw[j].z, bw[j].w});
        acc[i][j] = mfma_fp8(a0, b0, acc[i][j]);
        acc[i][j] = mfma_fp8(a1, b1, acc[i][j]);
      }
    }
  }
  for (int i = 0; i < 2; ++i) {
    for (int j = 0; j < 2; ++j) {
      const uint32_t n = (T0 + j) * 16 + lane % 16;
      for (int r = 0; r < 4; ++r) {
        const uint32_t m = m0 + i * 16 + 4 * (lane / 16) + r;
        if (m < a.m && n < a.n) {
          const float v = a.alpha * ((a.xs[m] * a.scales[n]) * acc[i][j][r]);
          if (a.y_f32) {
            static_cast<float *>(a.y)[uint64_t(m) * a.ldy + n] = v;
          } else {
            static_cast<uint16_t *>(a.y)[uint64_t(m) * a.ldy + n] = f32_to_bf16(v);
          }
        }
      }
    }
  }
}

}  // namespace

hipError_t launch_fp8_gemm(const uint8_t *xq, const float *xs, uint64_t ldxq,
                           const ullm_linear_weight_t *w, uint32_t m, void *y,
                           uint64_t ldy, bool y_f32, float alpha,
                           hipStream_t s) {
  GemmArgs a{};
  a.xq = xq;
  a.xs = xs;
  a.tiles = static_cast<const uint8_t *>(w->tiles);
  a.scales = static_cast<const float *>(w->aux);
  a.y = y;
  a.ldxq = ldxq;
  a.ldy = ldy;
  a.m = m;
  a.n = static_cast<uint32_t>(w->n);
  a.k = static_cast<uint32_t>(w->k);
  a.units = static_cast<uint32_t>(w->fp8.blocks_per_stripe());
  a.alpha = alpha;
  a.y_f32 = y_f32;
  const bool vec = reinterpret_cast<uintptr_t>(xq) % 16 == 0 && ldxq % 16 == 0;
  const dim3 grid((a.n + 63) / 64, (m + 63) / 64);
  hipLaunchKernelGGL(fp8_gemm_direct_kernel, grid, dim3(256), 0, s, a, vec);
  return hipGetLastError();
}

}  // namespace ullm
