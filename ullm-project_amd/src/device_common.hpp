// device_common.hpp -- gfx950 device helpers shared by the linear kernels.
//
// Number formats follow the definitions of the quantized linear path:
// OCP E4M3FN (bias 7, max 448, NaN 0x7F, saturating RNE encode), bf16 RNE,
// IEEE f16.  Every conversion here is exact or round-to-nearest-even and
// must agree bit for bit with the CPU oracle used by the tests.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ullm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
typedef short s16x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---------------------------------------------------------------- bit casts
__device__ __forceinline__ uint32_t f32_bits(float x) {
  return __builtin_bit_cast(uint32_t, x);
}
__device__ __forceinline__ float bits_f32(uint32_t b) {
  return __builtin_bit_cast(float, b);
}

// bf16 <-> f32.  Decode is a shift.  Encode is round-to-nearest-even on the
// 16 dropped bits, with NaN kept quiet (sign and upper payload kept, bit 6
// set) and overflow carrying into infinity: gfx950's v_cvt_pk_bf16_f32, two
// values per instruction.  That instruction equals this rule bit for bit on
// all 2^32 inputs, denormals included (with f32 denormals enabled, as this
// library is built); ullm_bench_bf16_convert_check re-checks it on a device.
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return bits_f32(static_cast<uint32_t>(h) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
}
// lo in bits 0..15, hi in bits 16..31.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{lo, hi}, b2));
}

// f16 <-> f32 through the hardware converts (RNE, f16 denormals preserved).
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
__device__ __forceinline__ uint16_t f32_to_f16(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

// E4M3FN decode from the format definition: exponent field 0 is subnormal
// (m * 2^-9), otherwise (8 + m) * 2^(e - 10).  0x7F/0xFF are NaN.
__device__ __forceinline__ float e4m3_to_f32(uint32_t code) {
  const uint32_t mag = code & 0x7fu;
  const uint32_t e = mag >> 3;
  const uint32_t m = mag & 7u;
  float v;
  if (mag == 0x7fu) {
    v = __builtin_nanf("");
  } else if (e == 0) {
    v = static_cast<float>(m) * 0.001953125f;  // 2^-9
  } else {
    // 2^(e-7) * (1 + m/8): rebias the exponent into f32 (127 - 7 = 120).
    v = bits_f32(((e + 120u) << 23) | (m << 20));
  }
  return (code & 0x80u) ? -v : v;
}

// E4M3FN encode: RNE on the 20 dropped mantissa bits of an f32 in the normal
// range, quantum 2^-9 below 2^-6, and saturation of |x| >= 448 to 448.
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
  const uint32_t b = f32_bits(x);
  const uint32_t sign = (b >> 24) & 0x80u;
  const uint32_t a = b & 0x7fffffffu;
  if (a > 0x7f800000u) {
    return sign | 0x7fu;
  }
  if (a >= 0x43e00000u) {  // 448.0f
    return sign | 0x7eu;
  }
  if (a < 0x3c800000u) {  // 2^-6: multiples of 2^-9, 8 * 2^-9 is code 0x08
    const float v = bits_f32(a) * 512.0f;
    return sign | static_cast<uint32_t>(__builtin_rintf(v));
  }
  const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
  return sign | ((r >> 20) - (120u << 3));
}

// ------------------------------------------------------------ MFMA helpers
// v_mfma_f32_16x16x32_bf16: src0 lane l carries row (l % 16), k-slots
// 8*(l/16)..+7; src1 lane l carries column (l % 16) for the same k-slots;
// the result lane l holds rows 4*(l/16)+r, column l % 16, r = 0..3.
__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Four E4M3 codes in one dword -> four bf16 (exact: every E4M3 value is a
// bf16 value).  Scale 1.0 makes the scaled convert a plain convert.
__device__ __forceinline__ u32x2 e4m3x4_to_bf16x4(uint32_t w) {
  const bf16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
  const bf16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
  u32x2 r;
  r.x = __builtin_bit_cast(uint32_t, lo);
  r.y = __builtin_bit_cast(uint32_t, hi);
  return r;
}

// Eight 4-bit codes in one dword -> eight bf16 holding 128 + q, exact because
// 128..143 need 8 significant bits.  Element t of the result is nibble
// (t / 2) + 4 * (t % 2) of w: inserting a nibble into the low mantissa bits
// of bf16 128.0 (0x4300) yields 128 + q.  `mask` (0x000f000f) and `magic`
// (0x43004300) come from opaque_u32() so they live in registers and each
// insert compiles to one v_bfi_b32 (gfx9 VOP3 takes no literal operands).
__device__ __forceinline__ bf16x8 nib8_to_bf16_off128(uint32_t w,
                                                      uint32_t mask,
                                                      uint32_t magic) {
  u32x4 r;
  r.x = (w & mask) | (magic & ~mask);
  r.y = ((w >> 4) & mask) | (magic & ~mask);
  r.z = ((w >> 8) & mask) | (magic & ~mask);
  r.w = ((w >> 12) & mask) | (magic & ~mask);
  return __builtin_bit_cast(bf16x8, r);
}

// A constant the compiler cannot fold into instructions (kept in a VGPR).
__device__ __forceinline__ uint32_t opaque_u32(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

__device__ __forceinline__ bf16x8 nib8_to_bf16_off128(uint32_t w) {
  return nib8_to_bf16_off128(w, 0x000f000fu, 0x43004300u);
}

// Nibble position inside a device AQ4 word for MFMA element t (inverse of the
// mapping in nib8_to_bf16_off128).
__host__ __device__ constexpr uint32_t aq4_nibble_pos(uint32_t t) {
  return (t >> 1) + 4u * (t & 1u);
}

// ------------------------------------------------------- wave reductions
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    v = fmaxf(v, __shfl_xor(v, off, kWave));
  }
  return v;
}
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    v = fminf(v, __shfl_xor(v, off, kWave));
  }
  return v;
}

// Byte-range buffer over device memory: loads at offsets past `bytes` return
// zero without a memory access, which lets a software pipeline issue its
// look-ahead loads unconditionally (a branch around a load makes the compiler
// drain every outstanding load at the join).  Offsets are 32-bit: the range
// must stay below 2 GiB.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t byte_buffer(const void *p,
                                                             uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0,
                                           static_cast<int>(bytes), 0x00020000);
}
constexpr int kNt = 2;                      // nontemporal cache policy bit

// ------------------------------------------------------------ epilogues
// What the linear kernels do with an output element after alpha is applied.
enum : uint32_t {
  kEpiNone = 0,      // y = v
  kEpiSiluMul = 1,   // gated-pair weight: y[:, j] = silu(gate_j) * up_j
  kEpiResidual = 2,  // y = v + r (r may be y itself)
};
struct Epilogue {
  uint32_t kind;
  uint32_t n_out;    // output columns: N, or F = N / 2 for kEpiSiluMul
  const void *res;   // kEpiResidual: r [m][ldr], bf16 or f32
  uint64_t ldr;
  bool res_f32;
};

// silu(g) = g * sigmoid(g) = g / (1 + e^-g), in fp32.
__device__ __forceinline__ float silu_f32(float g) {
  return g / (1.0f + expf(-g));
}

// Store output element (m, p): p is the column in the weight's physical row
// order (its tile layout), n the weight's logical row count, v the value
// with alpha applied, ok whether row m exists (and the column's stripe is
// live).  Every lane of a wave must reach this call in the same control flow
// with its own (m, p) and the (m, p ^ 8) partner in lane ^ 8, as the MFMA
// output layout places them: kEpiSiluMul takes the up product from there.
// EPI is the epilogue kind, a compile-time constant so that the plain
// kernels carry no epilogue code (it sits inside their streaming loops).
template <uint32_t EPI>
__device__ __forceinline__ void store_out(void *y, uint64_t ldy, bool y_f32,
                                          const Epilogue &e, uint32_t n,
                                          uint32_t m, uint32_t p, float v,
                                          bool ok) {
  uint32_t col = p;
  if constexpr (EPI == kEpiSiluMul) {
    const float up = __shfl_xor(v, 8, kWave);
    col = (p / 16) * 8 + p % 16;
    ok = ok && p % 16 < 8 && col < e.n_out;
    v = silu_f32(v) * up;
  } else {
    ok = ok && p < n;
    if (EPI == kEpiResidual && ok) {
      const uint64_t i = uint64_t(m) * e.ldr + p;
      v += e.res_f32 ? static_cast<const float *>(e.res)[i]
                     : bf16_to_f32(static_cast<const uint16_t *>(e.res)[i]);
    }
  }
  if (ok) {
    if (y_f32) {
      static_cast<float *>(y)[uint64_t(m) * ldy + col] = v;
    } else {
      static_cast<uint16_t *>(y)[uint64_t(m) * ldy + col] = f32_to_bf16(v);
    }
  }
}

}  // namespace ullm
