// layout.hpp -- HBM layout of device-resident quantized weights.
//
// The ABI exchanges weights in the canonical row-major encodings declared in
// include/ullm/linear.h.  In HBM they are repacked into "wave tiles": 1 KiB
// blocks that one 64-lane wavefront fetches with a single 16-byte-per-lane
// load, lane l receiving exactly the operand bytes it feeds to
// v_mfma_f32_16x16x32_bf16 as the B (weight) matrix.  Every weight load of the
// decode kernels is therefore one fully coalesced 1 KiB transaction, and the
// tiles of one 16-row stripe are contiguous along K.
//
// FP8 (E4M3, per-row f32 scale):
//   n16 = roundup(N, 16), k64 = roundup(K, 64), padding bytes are 0.
//   stripe T = n / 16, block b = k / 64, lane l = (n % 16) + 16 * ((k % 64) / 16),
//   byte  = k % 16;  offset = ((T * (k64 / 64) + b) * 64 + l) * 16 + byte.
//   Lane bytes 0..7 feed one MFMA (k-slots 0..7 of the lane), bytes 8..15 the
//   next, so lane l of a block covers k = 64b + 16*(l/16) .. +15 of row n.
//   scales: f32 [n16], padding 0.
//
// AQ4 (g128, f16 scale + f16 zero):
//   n16 = roundup(N, 16), K % 128 == 0, groups G = K / 128.
//   tile (T, g) is 64 lanes x 4 dwords; lane l = (n % 16) + 16 * q4, dword j.
//   dword (T, g, l, j) holds the 8 codes of row n at k = 128g + 32j + 8*q4 + t,
//   t = 0..7, with code t at nibble aq4_nibble_pos(t).  Dword j feeds the j-th
//   MFMA of the group.  dword offset = ((T * G + g) * 64 + l) * 4 + j.
//   scale/zero: u32 [(T * G + g) * 16 + n % 16] = f16 scale | f16 zero << 16.
//
// Row placement.  Above, n is the weight's physical row p(n).  For a plain
// weight p(n) = n.  A gated-pair weight (N = 2F rows: F gate rows, then the F
// matching up rows of a fused gate/up projection) interleaves the two halves
// in blocks of 8: physical stripe T holds gate rows 8T..8T+7 in its rows 0..7
// and up rows 8T..8T+7 in rows 8..15, so each output feature's gate and up
// products come out of the same MFMA tile in lanes l and l ^ 8, and n16 =
// 2 * roundup(F, 8).  Unmapped physical rows stay zero.
#pragma once

#include <stdint.h>

namespace ullm {

__host__ __device__ constexpr uint64_t round_up(uint64_t v, uint64_t m) {
  return (v + m - 1) / m * m;
}

// Physical row of canonical row n (gate = F for a gated-pair weight, else 0).
__host__ __device__ constexpr uint64_t phys_row(uint64_t n, uint64_t gate) {
  return gate == 0   ? n
         : n < gate  ? (n / 8) * 16 + n % 8
                     : ((n - gate) / 8) * 16 + 8 + (n - gate) % 8;
}
__host__ __device__ constexpr uint64_t phys_rows(uint64_t n, uint64_t gate) {
  return gate == 0 ? round_up(n, 16) : 2 * round_up(gate, 8);
}

struct Fp8Layout {
  uint64_t n, k, n16, k64;
  uint64_t gate;  // F of a gated-pair weight, 0 for a plain one
  __host__ __device__ uint64_t phys(uint64_t row) const { return phys_row(row, gate); }
  __host__ __device__ uint64_t blocks_per_stripe() const { return k64 / 64; }
  __host__ __device__ uint64_t bytes() const { return n16 * k64; }
  // Byte of canonical element (row, col).
  __host__ __device__ uint64_t offset(uint64_t row, uint64_t col) const {
    row = phys(row);
    const uint64_t lane = (row % 16) + 16 * ((col % 64) / 16);
    return (((row / 16) * blocks_per_stripe() + col / 64) * 64 + lane) * 16 +
           col % 16;
  }
};

struct Aq4Layout {
  uint64_t n, k, n16, groups;
  uint64_t gate;  // F of a gated-pair weight, 0 for a plain one
  __host__ __device__ uint64_t phys(uint64_t row) const { return phys_row(row, gate); }
  __host__ __device__ uint64_t words() const { return n16 * groups * 256; }
  __host__ __device__ uint64_t sz_words() const { return n16 * groups; }
};

// gate: F = n / 2 for a gated-pair weight (n even), 0 for a plain one.
inline Fp8Layout make_fp8_layout(uint64_t n, uint64_t k, uint64_t gate = 0) {
  return Fp8Layout{n, k, phys_rows(n, gate), round_up(k, 64), gate};
}
inline Aq4Layout make_aq4_layout(uint64_t n, uint64_t k, uint64_t gate = 0) {
  return Aq4Layout{n, k, phys_rows(n, gate), k / 128, gate};
}

}  // namespace ullm
