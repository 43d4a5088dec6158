// kernels.hpp -- host-side launchers of the gfx950 kernels.  Each launcher
// checks nothing beyond what its kernel's indexing assumes (the C-ABI layer
// validates user input first) and returns the launch status.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device_common.hpp"
#include "layout.hpp"

namespace ullm {

// ---------------------------------------------------------------- weights
hipError_t launch_fp8_quantize(const float *w, const Fp8Layout &L,
                               uint8_t *tiles, float *scales, hipStream_t s);
hipError_t launch_fp8_pack(const uint8_t *q, const float *scales_in,
                           const Fp8Layout &L, uint8_t *tiles, float *scales,
                           hipStream_t s);
hipError_t launch_fp8_export(const uint8_t *tiles, const float *scales,
                             const Fp8Layout &L, uint8_t *q, float *s_out,
                             hipStream_t s);
hipError_t launch_fp8_dequant(const uint8_t *tiles, const float *scales,
                              const Fp8Layout &L, float *out, hipStream_t s);

hipError_t launch_aq4_quantize(const float *w, const Aq4Layout &L,
                               uint32_t *tiles, uint32_t *sz, hipStream_t s);
hipError_t launch_aq4_pack(const uint32_t *packed, const uint16_t *scales,
                           const uint16_t *zeros, const Aq4Layout &L,
                           uint32_t *tiles, uint32_t *sz, hipStream_t s);
hipError_t launch_aq4_export(const uint32_t *tiles, const uint32_t *sz,
                             const Aq4Layout &L, uint32_t *packed,
                             uint16_t *scales, uint16_t *zeros, hipStream_t s);
hipError_t launch_aq4_dequant(const uint32_t *tiles, const uint32_t *sz,
                              const Aq4Layout &L, float *out, hipStream_t s);

// ------------------------------------------------------------ activations
hipError_t launch_act_quant(const uint16_t *x, uint64_t ldx, uint64_t m,
                            uint64_t k, uint8_t *xq, float *xs, hipStream_t s);

// ------------------------------------------------------------------ GEMV
struct GemvArgs {
  const void *tiles;   // device weight tiles (Fp8Layout / Aq4Layout)
  const void *aux;     // FP8: f32 scales [n16]; AQ4: u32 scale|zero words
  const uint16_t *x;   // bf16 [m][ldx]
  void *y;             // bf16 or f32 [m][ldy]
  uint64_t ldx, ldy;
  uint32_t m, n, k;    // logical sizes
  uint32_t n16;        // padded rows
  uint32_t units;      // FP8: k64 / 64; AQ4: k / 128
  float alpha;
  bool y_f32;
  uint32_t spw;        // stripes per workgroup (multi-stripe kernels; set by the launcher)
  Epilogue epi;        // output epilogue (n_out = output columns)
  // Split-K scratch (null = no split): counters, zero on entry and left zero,
  // and fp32 partial sums; the launcher sets ksplit.
  uint32_t *cnt;
  float *part;
  uint32_t ksplit;
};
hipError_t launch_fp8_gemv(const GemvArgs &a, hipStream_t s);
hipError_t launch_aq4_gemv(const GemvArgs &a, hipStream_t s);
// Bytes of split-K scratch the launch for these arguments would use (0: it
// does not split).  The first bytes are counters that must be zero.
uint64_t gemv_scratch_bytes(const GemvArgs &a, bool aq4);
// Offset of the partial sums inside that scratch.
uint64_t gemv_scratch_part_offset(const GemvArgs &a);

}  // namespace ullm
