// weights.hip -- quantization, repacking, export and dequantization of
// device-resident weights, and per-token activation quantization.
//
// These kernels run once per weight (creation) or are parity/debug tools; the
// activation quantizer is on the prefill path and is HBM-bound (2 bytes read,
// 1 byte written per element).  All arithmetic that defines a quantized value
// is written with FMA contraction off so it matches the format definitions
// bit for bit: q = enc(w / s), dequant = dec(q) * s, AQ4 dequant = (q - z) * s.
#include "device_common.hpp"
#include "kernels.hpp"

#pragma clang fp contract(off)

namespace ullm {
namespace {

constexpr int kBlock = 256;

template <int BLOCK = kBlock>
__device__ float block_max(float v, float *red) {
  v = wave_max(v);
  const int wave = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) {
    red[wave] = v;
  }
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < BLOCK / kWave; ++i) {
    r = fmaxf(r, red[i]);
  }
  return r;
}

// --------------------------------------------------------------- FP8 rows
// One workgroup per weight row: s = max|w| / 448, q = e4m3(w / s).
__global__ __launch_bounds__(kBlock) void fp8_quantize_kernel(
    const float *__restrict__ w, Fp8Layout L, uint8_t *__restrict__ tiles,
    float *__restrict__ scales) {
  __shared__ float red[kBlock / kWave];
  const uint64_t row = blockIdx.x;
  const float *src = w + row * L.k;
  float amax = 0.0f;
  for (uint64_t c = threadIdx.x; c < L.k; c += kBlock) {
    amax = fmaxf(amax, fabsf(src[c]));
  }
  amax = block_max(amax, red);
  const float s = amax / 448.0f;
  if (threadIdx.x == 0) {
    scales[L.phys(row)] = s;
  }
  for (uint64_t c = threadIdx.x; c < L.k; c += kBlock) {
    const uint32_t q = s == 0.0f ? 0u : f32_to_e4m3(src[c] / s);
    tiles[L.offset(row, c)] = static_cast<uint8_t>(q);
  }
}

__global__ __launch_bounds__(kBlock) void fp8_pack_kernel(
    const uint8_t *__restrict__ q, const float *__restrict__ s_in, Fp8Layout L,
    uint8_t *__restrict__ tiles, float *__restrict__ scales) {
  const uint64_t total = L.n * L.k;
  for (uint64_t i = blockIdx.x * uint64_t(kBlock) + threadIdx.x; i < total;
       i += uint64_t(gridDim.x) * kBlock) {
    const uint64_t row = i / L.k, col = i % L.k;
    tiles[L.offset(row, col)] = q[i];
    if (col == 0) {
      scales[L.phys(row)] = s_in[row];
    }
  }
}

__global__ __launch_bounds__(kBlock) void fp8_export_kernel(
    const uint8_t *__restrict__ tiles, const float *__restrict__ scales,
    Fp8Layout L, uint8_t *__restrict__ q, float *__restrict__ s_out) {
  const uint64_t total = L.n * L.k;
  for (uint64_t i = blockIdx.x * uint64_t(kBlock) + threadIdx.x; i < total;
       i += uint64_t(gridDim.x) * kBlock) {
    const uint64_t row = i / L.k, col = i % L.k;
    q[i] = tiles[L.offset(row, col)];
    if (col == 0) {
      s_out[row] = scales[L.phys(row)];
    }
  }
}

__global__ __launch_bounds__(kBlock) void fp8_dequant_kernel(
    const uint8_t *__restrict__ tiles, const float *__restrict__ scales,
    Fp8Layout L, float *__restrict__ out) {
  const uint64_t total = L.n * L.k;
  for (uint64_t i = blockIdx.x * uint64_t(kBlock) + threadIdx.x; i < total;
       i += uint64_t(gridDim.x) * kBlock) {
    const uint64_t row = i / L.k, col = i % L.k;
    out[i] = e4m3_to_f32(tiles[L.offset(row, col)]) * scales[L.phys(row)];
  }
}

// ---------------------------------------------------------------- AQ4 g128
// Dword and scale|zero word of canonical row `row` (placed at its physical
// row).
__device__ __forceinline__ uint64_t aq4_word(const Aq4Layout &L, uint64_t row,
                                             uint64_t g, uint32_t q4,
                                             uint32_t j) {
  const uint64_t p = L.phys(row);
  return (((p / 16) * L.groups + g) * 64 + (p % 16) + 16 * q4) * 4 + j;
}
__device__ __forceinline__ uint64_t aq4_sz(const Aq4Layout &L, uint64_t row,
                                           uint64_t g) {
  const uint64_t p = L.phys(row);
  return ((p / 16) * L.groups + g) * 16 + p % 16;
}

// One wavefront per (row, group of 128).
__global__ __launch_bounds__(kWave) void aq4_quantize_kernel(
    const float *__restrict__ w, Aq4Layout L, uint32_t *__restrict__ tiles,
    uint32_t *__restrict__ sz) {
  __shared__ uint8_t codes[128];
  const uint64_t g = blockIdx.x;
  const uint64_t row = blockIdx.y;
  const uint32_t lane = threadIdx.x;
  const float *src = w + row * L.k + g * 128;
  const float v0 = src[lane];
  const float v1 = src[lane + 64];
  const float lo = wave_min(fminf(v0, v1));
  const float hi = wave_max(fmaxf(v0, v1));
  uint16_t s16 = f32_to_f16((hi - lo) / 15.0f);
  float sf = f16_to_f32(s16);
  uint16_t z16 = sf != 0.0f ? f32_to_f16(-lo / sf) : uint16_t(0);
  if (sf == 0.0f || !__builtin_isfinite(f16_to_f32(z16))) {
    s16 = 0x3c00u;  // 1.0
    z16 = f32_to_f16(-lo);
    sf = 1.0f;
  }
  const float zf = f16_to_f32(z16);
  const float u0 = __builtin_rintf(v0 / sf + zf);
  const float u1 = __builtin_rintf(v1 / sf + zf);
  codes[lane] = static_cast<uint8_t>(fminf(fmaxf(u0, 0.0f), 15.0f));
  codes[lane + 64] = static_cast<uint8_t>(fminf(fmaxf(u1, 0.0f), 15.0f));
  __syncthreads();
  if (lane < 16) {
    const uint32_t q4 = lane / 4, j = lane % 4;
    uint32_t word = 0;
#pragma unroll
    for (uint32_t t = 0; t < 8; ++t) {
      word |= uint32_t(codes[32 * j + 8 * q4 + t]) << (4 * aq4_nibble_pos(t));
    }
    tiles[aq4_word(L, row, g, q4, j)] = word;
  }
  if (lane == 0) {
    sz[aq4_sz(L, row, g)] = uint32_t(s16) | (uint32_t(z16) << 16);
  }
}

// One thread per canonical dword (row, w): the 8 codes k = 8w .. 8w+7 form
// exactly one device dword, with nibbles permuted to MFMA element order.
__global__ __launch_bounds__(kBlock) void aq4_pack_kernel(
    const uint32_t *__restrict__ packed, const uint16_t *__restrict__ scales,
    const uint16_t *__restrict__ zeros, Aq4Layout L,
    uint32_t *__restrict__ tiles, uint32_t *__restrict__ sz) {
  const uint64_t wpr = L.k / 8;
  const uint64_t total = L.n * wpr;
  for (uint64_t i = blockIdx.x * uint64_t(kBlock) + threadIdx.x; i < total;
       i += uint64_t(gridDim.x) * kBlock) {
    const uint64_t row = i / wpr, w = i % wpr;
    const uint64_t g = w / 16;
    const uint32_t j = (w % 16) / 4, q4 = w % 4;
    const uint32_t src = packed[i];
    uint32_t word = 0;
#pragma unroll
    for (uint32_t t = 0; t < 8; ++t) {
      word |= ((src >> (4 * t)) & 0xfu) << (4 * aq4_nibble_pos(t));
    }
    tiles[aq4_word(L, row, g, q4, j)] = word;
    if (w % 16 == 0) {
      const uint64_t si = row * L.groups + g;
      sz[aq4_sz(L, row, g)] = uint32_t(scales[si]) | (uint32_t(zeros[si]) << 16);
    }
  }
}

__global__ __launch_bounds__(kBlock) void aq4_export_kernel(
    const uint32_t *__restrict__ tiles, const uint32_t *__restrict__ sz,
    Aq4Layout L, uint32_t *__restrict__ packed, uint16_t *__restrict__ scales,
    uint16_t *__restrict__ zeros) {
  const uint64_t wpr = L.k / 8;
  const uint64_t total = L.n * wpr;
  for (uint64_t i = blockIdx.x * uint64_t(kBlock) + threadIdx.x; i < total;
       i += uint64_t(gridDim.x) * kBlock) {
    const uint64_t row = i / wpr, w = i % wpr;
    const uint64_t g = w / 16;
    const uint32_t j = (w % 16) / 4, q4 = w % 4;
    const uint32_t dev = tiles[aq4_word(L, row, g, q4, j)];
    uint32_t word = 0;
#pragma unroll
    for (uint32_t t = 0; t < 8; ++t) {
      word |= ((dev >> (4 * aq4_nibble_pos(t))) & 0xfu) << (4 * t);
    }
    packed[i] = word;
    if (w % 16 == 0) {
      const uint32_t v = sz[aq4_sz(L, row, g)];
      scales[row * L.groups + g] = uint16_t(v & 0xffffu);
      zeros[row * L.groups + g] = uint16_t(v >> 16);
    }
  }
}

__global__ __launch_bounds__(kBlock) void aq4_dequant_kernel(
    const uint32_t *__restrict__ tiles, const uint32_t *__restrict__ sz,
    Aq4Layout L, float *__restrict__ out) {
  const uint64_t total = L.n * L.k;
  for (uint64_t i = blockIdx.x * uint64_t(kBlock) + threadIdx.x; i < total;
       i += uint64_t(gridDim.x) * kBlock) {
    const uint64_t row = i / L.k, col = i % L.k;
    const uint64_t g = col / 128;
    const uint32_t kk = col % 128;
    const uint32_t j = kk / 32, q4 = (kk % 32) / 8, t = kk % 8;
    const uint32_t dev = tiles[aq4_word(L, row, g, q4, j)];
    const uint32_t code = (dev >> (4 * aq4_nibble_pos(t))) & 0xfu;
    const uint32_t v = sz[aq4_sz(L, row, g)];
    const float sf = f16_to_f32(uint16_t(v & 0xffffu));
    const float zf = f16_to_f32(uint16_t(v >> 16));
    out[i] = (float(code) - zf) * sf;
  }
}

// ------------------------------------------------------ activation quant
// Optional fused addend: the quantized activations are x + b, each element
// the fp32 sum of the two bf16 values rounded to bf16 (round to nearest
// even), also written to `sum` when it is not null (`sum` may be x or b
// itself: every element is read before the same thread writes it).
struct AddIn {
  const uint16_t *b = nullptr;  // null: no addend
  uint64_t ldb = 0;
  uint16_t *sum = nullptr;
  uint64_t lds = 0;
};

__device__ __forceinline__ uint16_t add_bf16(uint16_t x, uint16_t y) {
  return f32_to_bf16(bf16_to_f32(x) + bf16_to_f32(y));
}

// One workgroup per token row: a = max|x| / 448, xq = e4m3(x / a).
template <bool ADD>
__global__ __launch_bounds__(kBlock) void act_quant_kernel(
    const uint16_t *x, uint64_t ldx, uint64_t k, uint8_t *__restrict__ xq,
    float *__restrict__ xs, AddIn add) {
  __shared__ float red[kBlock / kWave];
  const uint64_t row = blockIdx.x;
  const uint16_t *src = x + row * ldx;
  const uint16_t *bsrc = ADD ? add.b + row * add.ldb : nullptr;
  uint16_t *sdst = ADD && add.sum != nullptr ? add.sum + row * add.lds : nullptr;
  float amax = 0.0f;
  for (uint64_t c = threadIdx.x; c < k; c += kBlock) {
    uint16_t h = src[c];
    if constexpr (ADD) {
      h = add_bf16(h, bsrc[c]);
      if (sdst != nullptr) {
        sdst[c] = h;
      }
    }
    amax = fmaxf(amax, fabsf(bf16_to_f32(h)));
  }
  amax = block_max(amax, red);
  const float a = amax / 448.0f;
  if (threadIdx.x == 0) {
    xs[row] = a;
  }
  for (uint64_t c = threadIdx.x; c < k; c += kBlock) {
    // The sum written above is read back (it may have replaced x or b);
    // without a sum output it is formed again.
    const uint16_t h = !ADD ? src[c] : sdst != nullptr ? sdst[c] : add_bf16(src[c], bsrc[c]);
    const uint32_t q = a == 0.0f ? 0u : f32_to_e4m3(bf16_to_f32(h) / a);
    xq[row * k + c] = static_cast<uint8_t>(q);
  }
}

// Vectorized activation quantization for 16-byte aligned rows with K a
// multiple of 8: each thread keeps CH chunks of 8 bf16 of its row in
// registers (one 16-byte load each), so the row is read once, and writes 8
// codes per store.  The per-element arithmetic is that of act_quant_kernel.
// Workgroups of 256 threads, or 512 with the residual add (two input
// streams): measured on MI355X at M = 2048, K = 4096, the plain quantize
// takes 7.4 us with 256 threads against 8.3 with 512 and 8.1 with 128; the
// fused add 14.0 us with 512 against 14.8 with 256.
constexpr int kAddBlock = 512;
template <int CH, bool ADD>
__global__ __launch_bounds__(ADD ? kAddBlock : kBlock) void act_quant_vec_kernel(
    const uint16_t *x, uint64_t ldx, uint64_t k, uint8_t *__restrict__ xq,
    float *__restrict__ xs, AddIn add) {
  constexpr int kT = ADD ? kAddBlock : kBlock;
  __shared__ float red[kT / kWave];
  const uint64_t row = blockIdx.x;
  const uint16_t *src = x + row * ldx;
  u32x4 v[CH];
  // Row maximum of the bf16 magnitudes as integers: for non-NaN values the
  // bit order is the value order, and any inf or NaN shows as >= 0x7f80.
  u16x2 mx = {0, 0};
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const uint64_t idx = (uint64_t(c) * kT + threadIdx.x) * 8;
    v[c] = idx < k ? *reinterpret_cast<const u32x4 *>(src + idx)
                   : u32x4{0u, 0u, 0u, 0u};
    if constexpr (ADD) {
      if (idx < k) {
        const u32x4 b = *reinterpret_cast<const u32x4 *>(add.b + row * add.ldb + idx);
        u32x4 r;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          r[e] = f32x2_to_bf16x2(bits_f32(v[c][e] << 16) + bits_f32(b[e] << 16),
                                 bits_f32(v[c][e] & 0xffff0000u) +
                                     bits_f32(b[e] & 0xffff0000u));
        }
        v[c] = r;
        if (add.sum != nullptr) {
          *reinterpret_cast<u32x4 *>(add.sum + row * add.lds + idx) = r;
        }
      }
    }
    const uint32_t w[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      mx = __builtin_elementwise_max(
          mx, __builtin_bit_cast(u16x2, w[e] & 0x7fff7fffu));
    }
  }
  const uint32_t mb = mx.x > mx.y ? mx.x : mx.y;
  float amax = block_max<kT>(mb >= 0x7f80u ? __builtin_inff() : bits_f32(mb << 16), red);
  const bool finite = amax != __builtin_inff();
  if (!finite) {
    // A row holding inf or NaN: max|x| over the non-NaN values, as fmaxf.
    __syncthreads();
    float am = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const uint32_t w[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        am = fmaxf(am, fabsf(bf16_to_f32(uint16_t(w[e] & 0xffffu))));
        am = fmaxf(am, fabsf(bf16_to_f32(uint16_t(w[e] >> 16))));
      }
    }
    amax = block_max<kT>(am, red);
  }
  const float a = amax / 448.0f;
  if (threadIdx.x == 0) {
    xs[row] = a;
  }
  // x / a through the row's reciprocal: q0 = x * r, then one residual step
  // q = q0 + (x - q0 a) r with fused multiply-adds (r = 1 / a correctly
  // rounded, once per row).  For a >= 2^-100 this gives the same E4M3 code
  // as the correctly rounded quotient for every bf16 x with |x| <= max|x|:
  // checked exhaustively over every finite bf16 row maximum and every such
  // x (tests/test_act_quant_division.py).  The quotients that differ in the
  // last fp32 bit lie far below the smallest E4M3 code, and an exact zero
  // keeps its sign (q0).  Rows with a smaller scale divide.
  const float rcp = 1.0f / a;
  const bool via_rcp = a >= 0x1p-100f;
  auto quot = [&](float x) {
    if (!via_rcp) {
      return x / a;
    }
    const float q0 = x * rcp;
    const float q1 = __builtin_fmaf(__builtin_fmaf(-q0, a, x), rcp, q0);
    return q0 == 0.0f ? q0 : q1;
  };
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const uint64_t idx = (uint64_t(c) * kT + threadIdx.x) * 8;
    if (idx < k) {
      const uint32_t w[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
      uint32_t out[2] = {0u, 0u};
      if (finite && a != 0.0f) {
        // Every quotient is finite with |x / a| <= 448 (one rounding of
        // 448 at most above it), where the hardware E4M3 convert rounds to
        // nearest even exactly like f32_to_e4m3; scale 1.0 leaves it plain.
#pragma unroll
        for (int d = 0; d < 2; ++d) {
          float f[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t ww = w[2 * d + e / 2];
            f[e] = quot(bf16_to_f32(uint16_t(e % 2 ? ww >> 16 : ww & 0xffffu)));
          }
          s16x2 r = {0, 0};
          r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, f[0], f[1], 1.0f, false);
          r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, f[2], f[3], 1.0f, true);
          out[d] = __builtin_bit_cast(uint32_t, r);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint16_t h = uint16_t(e % 2 ? w[e / 2] >> 16 : w[e / 2] & 0xffffu);
          const uint32_t q = a == 0.0f ? 0u : f32_to_e4m3(bf16_to_f32(h) / a);
          out[e / 4] |= q << (8 * (e % 4));
        }
      }
      *reinterpret_cast<u32x2 *>(xq + row * k + idx) = u32x2{out[0], out[1]};
    }
  }
}

unsigned grid_for(uint64_t total) {
  const uint64_t blocks = (total + kBlock - 1) / kBlock;
  return static_cast<unsigned>(blocks < 65536 ? (blocks ? blocks : 1) : 65536);
}

}  // namespace

hipError_t launch_fp8_quantize(const float *w, const Fp8Layout &L,
                               uint8_t *tiles, float *scales, hipStream_t s) {
  hipLaunchKernelGGL(fp8_quantize_kernel, dim3(L.n), dim3(kBlock), 0, s, w, L,
                     tiles, scales);
  return hipGetLastError();
}

hipError_t launch_fp8_pack(const uint8_t *q, const float *scales_in,
                           const Fp8Layout &L, uint8_t *tiles, float *scales,
                           hipStream_t s) {
  hipLaunchKernelGGL(fp8_pack_kernel, dim3(grid_for(L.n * L.k)), dim3(kBlock),
                     0, s, q, scales_in, L, tiles, scales);
  return hipGetLastError();
}

hipError_t launch_fp8_export(const uint8_t *tiles, const float *scales,
                             const Fp8Layout &L, uint8_t *q, float *s_out,
                             hipStream_t s) {
  hipLaunchKernelGGL(fp8_export_kernel, dim3(grid_for(L.n * L.k)),
                     dim3(kBlock), 0, s, tiles, scales, L, q, s_out);
  return hipGetLastError();
}

hipError_t launch_fp8_dequant(const uint8_t *tiles, const float *scales,
                              const Fp8Layout &L, float *out, hipStream_t s) {
  hipLaunchKernelGGL(fp8_dequant_kernel, dim3(grid_for(L.n * L.k)),
                     dim3(kBlock), 0, s, tiles, scales, L, out);
  return hipGetLastError();
}

hipError_t launch_aq4_quantize(const float *w, const Aq4Layout &L,
                               uint32_t *tiles, uint32_t *sz, hipStream_t s) {
  hipLaunchKernelGGL(aq4_quantize_kernel, dim3(L.groups, L.n), dim3(kWave), 0,
                     s, w, L, tiles, sz);
  return hipGetLastError();
}

hipError_t launch_aq4_pack(const uint32_t *packed, const uint16_t *scales,
                           const uint16_t *zeros, const Aq4Layout &L,
                           uint32_t *tiles, uint32_t *sz, hipStream_t s) {
  hipLaunchKernelGGL(aq4_pack_kernel, dim3(grid_for(L.n * (L.k / 8))),
                     dim3(kBlock), 0, s, packed, scales, zeros, L, tiles, sz);
  return hipGetLastError();
}

hipError_t launch_aq4_export(const uint32_t *tiles, const uint32_t *sz,
                             const Aq4Layout &L, uint32_t *packed,
                             uint16_t *scales, uint16_t *zeros, hipStream_t s) {
  hipLaunchKernelGGL(aq4_export_kernel, dim3(grid_for(L.n * (L.k / 8))),
                     dim3(kBlock), 0, s, tiles, sz, L, packed, scales, zeros);
  return hipGetLastError();
}

hipError_t launch_aq4_dequant(const uint32_t *tiles, const uint32_t *sz,
                              const Aq4Layout &L, float *out, hipStream_t s) {
  hipLaunchKernelGGL(aq4_dequant_kernel, dim3(grid_for(L.n * L.k)),
                     dim3(kBlock), 0, s, tiles, sz, L, out);
  return hipGetLastError();
}

namespace {

template <bool ADD>
hipError_t launch_act_quant_t(const uint16_t *x, uint64_t ldx, uint64_t m,
                              uint64_t k, uint8_t *xq, float *xs,
                              const AddIn &add, hipStream_t s) {
  auto a16 = [](const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  bool vec = a16(x) && ldx % 8 == 0 && k % 8 == 0 &&
             reinterpret_cast<uintptr_t>(xq) % 8 == 0;
  if (ADD) {
    vec = vec && a16(add.b) && add.ldb % 8 == 0 &&
          (add.sum == nullptr || (a16(add.sum) && add.lds % 8 == 0));
  }
  const int threads = ADD ? kAddBlock : kBlock;
  const uint64_t chunks = (k / 8 + threads - 1) / threads;  // per thread
  if (vec && chunks <= 8) {
    auto kernel = chunks <= 1   ? act_quant_vec_kernel<1, ADD>
                  : chunks <= 2 ? act_quant_vec_kernel<2, ADD>
                  : chunks <= 4 ? act_quant_vec_kernel<4, ADD>
                                : act_quant_vec_kernel<8, ADD>;
    hipLaunchKernelGGL(kernel, dim3(m), dim3(threads), 0, s, x, ldx, k, xq, xs, add);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(act_quant_kernel<ADD>, dim3(m), dim3(kBlock), 0, s, x, ldx,
                     k, xq, xs, add);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_act_quant(const uint16_t *x, uint64_t ldx, uint64_t m,
                            uint64_t k, uint8_t *xq, float *xs, hipStream_t s) {
  return launch_act_quant_t<false>(x, ldx, m, k, xq, xs, AddIn{}, s);
}

hipError_t launch_add_act_quant(const uint16_t *x, uint64_t ldx,
                                const uint16_t *b, uint64_t ldb, uint16_t *sum,
                                uint64_t lds, uint64_t m, uint64_t k,
                                uint8_t *xq, float *xs, hipStream_t s) {
  AddIn add;
  add.b = b;
  add.ldb = ldb;
  add.sum = sum;
  add.lds = lds;
  return launch_act_quant_t<true>(x, ldx, m, k, xq, xs, add, s);
}

}  // namespace ullm
