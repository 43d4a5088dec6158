// gemv.hip -- decode-shape (M <= 32 per pass) quantized GEMV on gfx950.
//
// Y[m, n] = alpha * sum_k dequant(W)[n, k] * x[m, k], bf16 activations,
// fp32 accumulation, for FP8-E4M3 per-row-scaled and AQ4 g128 weights.
//
// The op is HBM-bound (intensity <= 64 flop/byte at M = 32 against a ridge of
// several hundred), so the kernel is built around streaming the weight tiles
// at full bandwidth and spending as few instructions as possible per byte:
//   * each weight load is one 1 KiB wave-tile (16 bytes per lane, see
//     layout.hpp), already in the lane order the matrix core consumes;
//   * the bytes are unpacked in registers straight into bf16 MFMA operands
//     (FP8 through the hardware scaled convert, AQ4 by OR-ing nibbles into the
//     mantissa of bf16 128.0) and contracted with v_mfma_f32_16x16x32_bf16
//     against bf16 activations read from L2 (x is tiny and shared by every
//     workgroup), so the ALU cost per weight byte is independent of M;
//   * one workgroup owns a 16-row stripe and one 32-row activation block; its
//     waves split K, each streaming a contiguous run of tiles with a batch of
//     loads in flight, and the partial sums meet in LDS once at the end.
// AQ4 uses the identity sum_k (q - z) s x = s * (sum_k (128 + q) x - (128 + z)
// sum_k x) per group: the integer codes stay exact in bf16, the group sum of x
// comes from a second MFMA against a ones operand, and the per-group scale and
// zero are applied once per 128 k in fp32.
#include "device_common.hpp"
#include "kernels.hpp"

namespace ullm {
namespace {

constexpr int kBatch = 8;  // tiles in flight per wave

// Eight (or sixteen) bf16 of activation row m starting at k0.  Rows beyond M
// and columns beyond K read as zero; `vec` says x rows are 16-byte aligned.
__device__ __forceinline__ bf16x8 load_x8(const uint16_t *__restrict__ xrow,
                                          bool valid, uint32_t k0, uint32_t K,
                                          bool vec) {
  u32x4 r = {0u, 0u, 0u, 0u};
  if (valid) {
    if (vec && k0 + 8 <= K) {
      r = *reinterpret_cast<const u32x4 *>(xrow + k0);
    } else {
      uint32_t h[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        h[i] = (k0 + i < K) ? xrow[k0 + i] : 0u;
      }
      r.x = h[0] | (h[1] << 16);
      r.y = h[2] | (h[3] << 16);
      r.z = h[4] | (h[5] << 16);
      r.w = h[6] | (h[7] << 16);
    }
  }
  return __builtin_bit_cast(bf16x8, r);
}

template <int MT, int WAVES>
__device__ __forceinline__ void reduce_and_store(const GemvArgs &a,
                                                 f32x4 (&acc)[MT], float *red,
                                                 const float *row_scale) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      red[((wave * MT + mt) * 4 + r) * kWave + lane] = acc[mt][r];
    }
  }
  __syncthreads();
  const uint32_t T = blockIdx.x;
  const uint32_t m_base = blockIdx.y * 32;
  for (int o = threadIdx.x; o < MT * 256; o += WAVES * kWave) {
    const int mt = o / 256;
    const int mrow = (o % 256) / 16;
    const int ncol = o % 16;
    const int src_lane = ncol + 16 * (mrow / 4);
    const int r = mrow % 4;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      v += red[((w * MT + mt) * 4 + r) * kWave + src_lane];
    }
    const uint32_t m = m_base + mt * 16 + mrow;
    const uint32_t n = T * 16 + ncol;
    if (m < a.m && n < a.n) {
      if (row_scale != nullptr) {
        v = row_scale[n] * v;
      }
      v = a.alpha * v;
      if (a.y_f32) {
        static_cast<float *>(a.y)[uint64_t(m) * a.ldy + n] = v;
      } else {
        static_cast<uint16_t *>(a.y)[uint64_t(m) * a.ldy + n] = f32_to_bf16(v);
      }
    }
  }
}

template <int MT, int WAVES>
__global__ __launch_bounds__(WAVES *kWave) void fp8_gemv_kernel(GemvArgs a,
                                                                bool vec) {
  __shared__ float red[WAVES * MT * 4 * kWave];
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const uint32_t T = blockIdx.x;
  const uint32_t units = a.units;
  const uint32_t ub = uint32_t(uint64_t(units) * wave / WAVES);
  const uint32_t ue = uint32_t(uint64_t(units) * (wave + 1) / WAVES);
  const uint8_t *stripe = static_cast<const uint8_t *>(a.tiles) +
                          uint64_t(T) * units * 1024 + lane * 16;

  const uint16_t *xrow[MT];
  bool valid[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const uint32_t m = blockIdx.y * 32 + mt * 16 + lane % 16;
    valid[mt] = m < a.m;
    xrow[mt] = a.x + uint64_t(valid[mt] ? m : 0) * a.ldx;
  }
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const uint32_t kl = 16 * (lane / 16);

  auto consume = [&](u32x4 wv, uint32_t u) {
    const u32x2 b01 = e4m3x4_to_bf16x4(wv.x);
    const u32x2 b23 = e4m3x4_to_bf16x4(wv.y);
    const u32x2 b45 = e4m3x4_to_bf16x4(wv.z);
    const u32x2 b67 = e4m3x4_to_bf16x4(wv.w);
    const bf16x8 b0 = __builtin_bit_cast(bf16x8, u32x4{b01.x, b01.y, b23.x, b23.y});
    const bf16x8 b1 = __builtin_bit_cast(bf16x8, u32x4{b45.x, b45.y, b67.x, b67.y});
    const uint32_t k0 = u * 64 + kl;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const bf16x8 a0 = load_x8(xrow[mt], valid[mt], k0, a.k, vec);
      const bf16x8 a1 = load_x8(xrow[mt], valid[mt], k0 + 8, a.k, vec);
      acc[mt] = mfma_bf16(a0, b0, acc[mt]);
      acc[mt] = mfma_bf16(a1, b1, acc[mt]);
    }
  };

  uint32_t u = ub;
  for (; u + kBatch <= ue; u += kBatch) {
    u32x4 wv[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      wv[i] = *reinterpret_cast<const u32x4 *>(stripe + uint64_t(u + i) * 1024);
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      consume(wv[i], u + i);
    }
  }
  for (; u < ue; ++u) {
    consume(*reinterpret_cast<const u32x4 *>(stripe + uint64_t(u) * 1024), u);
  }
  reduce_and_store<MT, WAVES>(a, acc, red,
                              static_cast<const float *>(a.aux));
}

template <int MT, int WAVES>
__global__ __launch_bounds__(WAVES *kWave) void aq4_gemv_kernel(GemvArgs a,
                                                                bool vec) {
  __shared__ float red[WAVES * MT * 4 * kWave];
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const uint32_t T = blockIdx.x;
  const uint32_t groups = a.units;
  const uint32_t ub = uint32_t(uint64_t(groups) * wave / WAVES);
  const uint32_t ue = uint32_t(uint64_t(groups) * (wave + 1) / WAVES);
  const uint32_t *stripe = static_cast<const uint32_t *>(a.tiles) +
                           uint64_t(T) * groups * 256 + lane * 4;
  const uint32_t *szs = static_cast<const uint32_t *>(a.aux) +
                        uint64_t(T) * groups * 16 + lane % 16;

  const uint16_t *xrow[MT];
  bool valid[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const uint32_t m = blockIdx.y * 32 + mt * 16 + lane % 16;
    valid[mt] = m < a.m;
    xrow[mt] = a.x + uint64_t(valid[mt] ? m : 0) * a.ldx;
  }
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const uint32_t kl = 8 * (lane / 16);
  const bf16x8 ones = __builtin_bit_cast(
      bf16x8, u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});

  auto consume = [&](u32x4 wv, uint32_t szv, uint32_t g) {
    const bf16x8 b[4] = {nib8_to_bf16_off128(wv.x), nib8_to_bf16_off128(wv.y),
                         nib8_to_bf16_off128(wv.z), nib8_to_bf16_off128(wv.w)};
    const float sf = f16_to_f32(uint16_t(szv & 0xffffu));
    const float zoff = 128.0f + f16_to_f32(uint16_t(szv >> 16));
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f32x4 p = {0.f, 0.f, 0.f, 0.f};
      f32x4 xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bf16x8 av =
            load_x8(xrow[mt], valid[mt], g * 128 + 32 * j + kl, a.k, vec);
        p = mfma_bf16(av, b[j], p);
        xs = mfma_bf16(av, ones, xs);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        acc[mt][r] += sf * (p[r] - zoff * xs[r]);
      }
    }
  };

  uint32_t g = ub;
  for (; g + kBatch <= ue; g += kBatch) {
    u32x4 wv[kBatch];
    uint32_t szv[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      wv[i] = *reinterpret_cast<const u32x4 *>(stripe + uint64_t(g + i) * 256);
      szv[i] = szs[uint64_t(g + i) * 16];
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      consume(wv[i], szv[i], g + i);
    }
  }
  for (; g < ue; ++g) {
    consume(*reinterpret_cast<const u32x4 *>(stripe + uint64_t(g) * 256),
            szs[uint64_t(g) * 16], g);
  }
  reduce_and_store<MT, WAVES>(a, acc, red, nullptr);
}

// Waves per workgroup: enough that the grid holds ~8 waves per CU on the
// 256-CU part, and no more waves than tile units to share out.
int pick_waves(uint64_t stripes, uint64_t mblocks, uint32_t units) {
  const uint64_t wgs = stripes * mblocks;
  int waves = 4;
  while (waves < 16 && wgs * waves < 2048 && uint32_t(waves * 2) <= units) {
    waves *= 2;
  }
  return waves;
}

template <int MT, int WAVES>
hipError_t launch_fp8_t(const GemvArgs &a, bool vec, hipStream_t s) {
  const dim3 grid(a.n16 / 16, (a.m + 31) / 32);
  hipLaunchKernelGGL((fp8_gemv_kernel<MT, WAVES>), grid, dim3(WAVES * kWave),
                     0, s, a, vec);
  return hipGetLastError();
}

template <int MT, int WAVES>
hipError_t launch_aq4_t(const GemvArgs &a, bool vec, hipStream_t s) {
  const dim3 grid(a.n16 / 16, (a.m + 31) / 32);
  hipLaunchKernelGGL((aq4_gemv_kernel<MT, WAVES>), grid, dim3(WAVES * kWave),
                     0, s, a, vec);
  return hipGetLastError();
}

bool x_vec_ok(const GemvArgs &a) {
  return (reinterpret_cast<uintptr_t>(a.x) % 16 == 0) && (a.ldx % 8 == 0);
}

}  // namespace

hipError_t launch_fp8_gemv(const GemvArgs &a, hipStream_t s) {
  const bool vec = x_vec_ok(a);
  const int waves = pick_waves(a.n16 / 16, (a.m + 31) / 32, a.units);
  const bool two = a.m > 16;
  switch (waves * 2 + (two ? 1 : 0)) {
    case 8: return launch_fp8_t<1, 4>(a, vec, s);
    case 9: return launch_fp8_t<2, 4>(a, vec, s);
    case 16: return launch_fp8_t<1, 8>(a, vec, s);
    case 17: return launch_fp8_t<2, 8>(a, vec, s);
    case 32: return launch_fp8_t<1, 16>(a, vec, s);
    default: return launch_fp8_t<2, 16>(a, vec, s);
  }
}

hipError_t launch_aq4_gemv(const GemvArgs &a, hipStream_t s) {
  const bool vec = x_vec_ok(a);
  const int waves = pick_waves(a.n16 / 16, (a.m + 31) / 32, a.units);
  const bool two = a.m > 16;
  switch (waves * 2 + (two ? 1 : 0)) {
    case 8: return launch_aq4_t<1, 4>(a, vec, s);
    case 9: return launch_aq4_t<2, 4>(a, vec, s);
    case 16: return launch_aq4_t<1, 8>(a, vec, s);
    case 17: return launch_aq4_t<2, 8>(a, vec, s);
    case 32: return launch_aq4_t<1, 16>(a, vec, s);
    default: return launch_aq4_t<2, 16>(a, vec, s);
  }
}

}  // namespace ullm
