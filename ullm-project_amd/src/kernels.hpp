// kernels.hpp -- host-side launchers of the gfx950 kernels.  Each launcher
// checks nothing beyond what its kernel's indexing assumes (the C-ABI layer
// validates user input first) and returns the launch status.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device_common.hpp"
#include "layout.hpp"
#include "ullm/linear.h"

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
// Per-token quantization of x + b (bf16 sums, optionally written to `sum`).
hipError_t launch_add_act_quant(const uint16_t *x, uint64_t ldx,
                                const uint16_t *b, uint64_t ldb, uint16_t *sum,
                                uint64_t lds, uint64_t m, uint64_t k,
                                uint8_t *xq, float *xs, hipStream_t s);

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
// K parts per stripe group that launch splits into (1: no split).
uint32_t gemv_split_parts(const GemvArgs &a, bool aq4);
// Offset of the partial sums inside that scratch.
uint64_t gemv_scratch_part_offset(const GemvArgs &a);
// Kernel family and shape a GEMV launch takes (the forward plan reports it).
// `split_ok`: split-K scratch is available (the plan assumes it is).
struct GemvChoice {
  uint32_t variant = 0;  // ULLM_LINEAR_GEMV_*
  uint32_t waves = 0;    // waves per workgroup
  uint32_t stripes = 1;  // register-staged: stripes sharing one activation load
  uint32_t classes = 1;  // activation row classes packed per MFMA A operand
  uint32_t ks = 1;       // split-K: K parts per stripe group
};
GemvChoice gemv_choice(const GemvArgs &a, bool aq4, bool split_ok);

// ------------------------------------------------------------------ GEMM
enum GemmKind : uint32_t {
  kGemmDirect = 0,      // operands straight from L2, 64 x 64 blocks
  kGemmLarge = 1,       // LDS-pipelined 256 x 256
  kGemmNarrow = 2,      // LDS-pipelined 256 x 224
  kGemmNarrow192 = 3,   // LDS-pipelined 256 x 192
  kGemmMid = 4,         // LDS-pipelined 128 x 128, two workgroups per CU
  kGemmNarrow128 = 5,   // LDS-pipelined 256 x 128
  kGemmNarrow64 = 6,    // LDS-pipelined 256 x 64
  kGemmSmall128 = 7,    // LDS-pipelined 128 x 64 (short prompts)
  kGemmSmall64 = 8,     // LDS-pipelined 64 x 64 (short prompts)
  kGemmSmall128W = 9,   // LDS-pipelined 128 x 128 (short prompts)
  kGemmSmall64W = 10,   // LDS-pipelined 64 x 128 (short prompts)
};
struct GemmPlan {
  uint32_t kind, block_m, block_n, tiles, grid;
  uint32_t ksplit;  // K parts per tile (1: no split); grid = tiles * ksplit
};
// The kernel and grid launch_fp8_gemm takes for an M x N x K product on a
// device of `cus` compute units (vec: activation rows 16-byte aligned;
// offsets_fit: operand offsets below 2^32).  grid < tiles means a
// persistent grid, each workgroup walking several tiles.
GemmPlan plan_fp8_gemm(uint32_t m, uint32_t n, uint32_t k, bool vec,
                       bool offsets_fit, uint32_t cus);
// The plan of a prefill call on the weight's device (xq: the quantized
// activations as the GEMM reads them, row stride ldxq bytes).
GemmPlan plan_fp8_gemm_call(const void *xq, uint64_t ldxq,
                            const ullm_linear_weight_t *w, uint32_t m);
// Split-K scratch of a plan: a counter region of kGemmCounterBytes (zero on
// entry, left zero) followed by the partial sums; 0 when it does not split.
constexpr uint64_t kGemmCounterBytes = 1024;
uint64_t gemm_split_bytes(const GemmPlan &p);

// ------------------------------------------------------------ host helpers
// Fixed device scratch of the allocation-free forward: a counter region
// (zero, and left zero by every launch) and a data region.
struct FixedScratch {
  char *counters;
  uint64_t counter_bytes;
  char *base;
  uint64_t bytes;
};
// Called with the weight's device current; fills *out or reports an error.
typedef ullm_status_t (*FixedScratchFn)(int device, hipStream_t stream,
                                        FixedScratch *out,
                                        ullm_error_sink_t *sink);
// ullm_linear_forward's body; `fixed` = null takes the caller's workspace or
// the library-owned buffers.
ullm_status_t forward_dispatch(const ullm_linear_forward_desc_t *desc,
                               ullm_error_sink_t *sink, FixedScratchFn fixed);

// Compute units of the current device, looked up once per device.
uint32_t device_cu_count();
// Launch-plan overrides for tuning sweeps.  Only a library built with
// -DULLM_TUNING reads them from the environment; the default build returns
// null for every name, so the launchers always take the configurations the
// parity tests cover.
const char *tuning_env(const char *name);

}  // namespace ullm
