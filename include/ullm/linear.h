/*
 * ullm/linear.h -- quantized linear-layer entry points (gfx950 build).
 *
 * The reference has no numerical linear layer: its Backend trait refuses
 * execution (reference crates/ullm-core/src/backend.rs:5-11,
 * crates/ullm-hip/src/lib.rs:510-512) and its Matmul descriptor checks shapes
 * only (crates/ullm-core/src/op.rs:97-113).  These functions are the native
 * side that HipBackend::execute would call for a Matmul whose B operand is an
 * FP8-row-scaled or AQ4 weight.  They follow the reference's ABI v1
 * conventions exactly (reference include/ullm/hip.h, native/hip/src/hip_stub.cpp):
 *   - every struct starts with {struct_size, abi_version}; a larger
 *     struct_size is accepted, a smaller one is ULLM_STATUS_INVALID_ARGUMENT
 *     (hip_stub.cpp:75-78), a wrong version ULLM_STATUS_INVALID_ABI_VERSION
 *     (hip_stub.cpp:79-82), non-zero reserved words
 *     ULLM_STATUS_RESERVED_NONZERO (hip_stub.cpp:94-98);
 *   - the error sink is validated first and reports like the v1 functions;
 *   - no C++ exception crosses the boundary (hip_stub.cpp:123,134);
 *   - handles are opaque, identity is checked against a live-handle table and
 *     a stale handle is ULLM_STATUS_HIP_INVALID_HANDLE
 *     (native/hip/src/hip_evidence_runtime.hip.cpp:276-303);
 *   - caller host memory is copied before a function returns and never kept
 *     (docs/architecture/runtime.md:77).
 *
 * Matrix conventions (all row-major, element strides):
 *   weight W[N][K]  (one output feature per row, K contiguous)
 *   activation X[M][K], output Y[M][N], Y = alpha * X * W^T.
 * Device memory is HIP device memory of the weight's device; streams are
 * hipStream_t passed as void* (null = the null stream).  Forward calls are
 * asynchronous in stream order.
 */
#ifndef ULLM_LINEAR_H
#define ULLM_LINEAR_H

#include "ullm/hip.h"

/* Extension statuses.  8..12 keep the values of the reference's private
 * evidence ABI (native/hip/src/evidence_abi.h:13-17); new codes start at 13. */
#ifndef ULLM_STATUS_HIP_TIMEOUT
#define ULLM_STATUS_HIP_TIMEOUT UINT32_C(8)
#define ULLM_STATUS_HIP_INVALID_HANDLE UINT32_C(9)
#define ULLM_STATUS_HIP_ZERO_DISPATCH UINT32_C(10)
#define ULLM_STATUS_HIP_RUNTIME_ERROR UINT32_C(11)
#define ULLM_STATUS_HIP_DISPATCH_CONTRACT UINT32_C(12)
#endif
#define ULLM_STATUS_OUT_OF_MEMORY UINT32_C(13)

/* Weight encodings.  The reference's Encoding enum (crates/ullm-core/src/
 * dtype.rs:55-66) has no variant for either; these are the values a future
 * Encoding::Fp8RowScaled / Encoding::Aq4 would map to. */
typedef uint32_t ullm_linear_encoding_t;
/* u8 E4M3FN codes [N][K] + f32 scale per row [N]. */
#define ULLM_LINEAR_ENCODING_FP8_E4M3_ROW UINT32_C(1)
/* u32 words [N][K/8] (nibble j of word w is k = 8w + j, low nibble first)
 * + f16 scale [N][K/128] + f16 zero [N][K/128]; K % 128 == 0. */
#define ULLM_LINEAR_ENCODING_AQ4_G128 UINT32_C(2)

/* Row layouts of a weight (ullm_linear_weight_desc_t.layout). */
#define ULLM_LINEAR_LAYOUT_PLAIN UINT32_C(0)
/* A fused gate/up projection: N = 2F rows, the F gate rows followed by the F
 * up rows of the same output features.  The library stores each feature's
 * gate and up rows side by side so that a forward with
 * ULLM_LINEAR_EPILOGUE_SILU_MUL produces Y[M][F] = silu(X Wg^T) * (X Wu^T)
 * in one pass.  Export and dequantize still use the canonical [2F][K] order. */
#define ULLM_LINEAR_LAYOUT_GATED_PAIRS UINT32_C(1)

/* Output epilogues (ullm_linear_forward_desc_t.epilogue), applied in fp32
 * after alpha, before the output is rounded. */
#define ULLM_LINEAR_EPILOGUE_NONE UINT32_C(0)
/* Gated-pair weight only: Y[m][j] = silu(a*g) * (a*u), g and u the gate and
 * up products of feature j, a = alpha, silu(v) = v / (1 + exp(-v)).  Y has
 * F = N / 2 columns. */
#define ULLM_LINEAR_EPILOGUE_SILU_MUL UINT32_C(1)
/* Y = alpha * X W^T + R for a residual R [M][N] (bf16 or f32).  R may be Y
 * itself (same pointer, dtype and row stride): an in-place residual add. */
#define ULLM_LINEAR_EPILOGUE_RESIDUAL_ADD UINT32_C(2)

/* What ullm_linear_weight_desc_t.values holds. */
#define ULLM_LINEAR_SOURCE_F32 UINT32_C(1)     /* f32 [N][K], quantized here */
#define ULLM_LINEAR_SOURCE_ENCODED UINT32_C(2) /* already-encoded buffers */

/* Where caller buffers live. */
#define ULLM_MEMORY_HOST UINT32_C(1)
#define ULLM_MEMORY_DEVICE UINT32_C(2)

/* Element types of activations and outputs (names as DType in
 * crates/ullm-core/src/dtype.rs:6-16). */
#define ULLM_LINEAR_DTYPE_BF16 UINT32_C(1)
#define ULLM_LINEAR_DTYPE_F32 UINT32_C(2)
#define ULLM_LINEAR_DTYPE_F8E4M3FN UINT32_C(3)

/* How bf16 activations enter the contraction. */
/* Exact: bf16 activations times dequantized weights, fp32 accumulation.
 * Any M; the decode kernels serve M <= 32 per weight pass. */
#define ULLM_LINEAR_ACT_EXACT UINT32_C(0)
/* Prefill: activations are quantized per token to E4M3 (scale = max|x|/448)
 * and contracted with FP8 weights on the FP8 matrix cores. */
#define ULLM_LINEAR_ACT_FP8_PER_TOKEN UINT32_C(1)

typedef struct ullm_linear_weight_t ullm_linear_weight_t;

typedef struct ullm_linear_weight_desc_t {
  uint32_t struct_size;
  uint32_t abi_version;
  uint32_t encoding; /* ULLM_LINEAR_ENCODING_* */
  uint32_t source;   /* ULLM_LINEAR_SOURCE_* */
  uint64_t n;        /* output features, >= 1 */
  uint64_t k;        /* input features, >= 1 (AQ4: multiple of 128) */
  uint32_t memory;   /* ULLM_MEMORY_* of values/scales/zeros */
  int32_t device;    /* HIP device ordinal that will own the weight */
  const void *values;
  const void *scales; /* ENCODED only */
  const void *zeros;  /* ENCODED AQ4 only */
  void *stream;       /* upload/quantize stream; creation blocks until done */
  uint32_t layout;    /* ULLM_LINEAR_LAYOUT_* (0 = plain) */
  uint32_t reserved0;
  uint64_t reserved[3];
} ullm_linear_weight_desc_t;

typedef struct ullm_linear_weight_info_t {
  uint32_t struct_size;
  uint32_t abi_version;
  uint32_t encoding;
  int32_t device;
  uint64_t n;
  uint64_t k;
  uint64_t device_bytes; /* bytes the weight holds in HBM */
  uint32_t layout;       /* ULLM_LINEAR_LAYOUT_* */
  uint32_t reserved0;
  uint64_t reserved[3];
} ullm_linear_weight_info_t;

typedef struct ullm_linear_forward_desc_t {
  uint32_t struct_size;
  uint32_t abi_version;
  const ullm_linear_weight_t *weight;
  uint64_t m;            /* rows of X and Y; 0 is a no-op */
  const void *x;         /* device, x_dtype [M][x_row_stride] */
  uint64_t x_row_stride; /* elements, 0 = K */
  const float *x_scales; /* device f32 [M]; required iff x_dtype is E4M3 */
  void *y;               /* device, y_dtype [M][y_row_stride] */
  uint64_t y_row_stride; /* elements, 0 = N */
  uint32_t x_dtype;      /* BF16, or F8E4M3FN (pre-quantized, FP8 weights) */
  uint32_t y_dtype;      /* BF16 (RNE) or F32 */
  uint32_t activation_mode; /* ULLM_LINEAR_ACT_*, for BF16 x */
  float alpha;              /* output multiplier; 1.0f for a plain product */
  void *stream;
  /* Device scratch (ullm_linear_workspace_size bytes) for prefill calls
   * (FP8 GEMM) and for split-K decode calls; null = library-owned.  Its
   * first 1 KiB holds split-K counters: zero it before the first use (every
   * call leaves that region zero, and no call writes it otherwise).  The
   * library-owned buffers are one per device and stream (calls on one stream
   * share them in stream order) and are allocated, or grown, by the first
   * call that needs them: make that call outside stream capture.  A grown
   * buffer's predecessor stays allocated, so graphs captured earlier remain
   * valid. */
  void *workspace;
  uint64_t workspace_size;
  uint32_t epilogue;            /* ULLM_LINEAR_EPILOGUE_* (0 = none) */
  uint32_t residual_dtype;      /* RESIDUAL_ADD: BF16 or F32 */
  const void *residual;         /* RESIDUAL_ADD: device [M][residual_row_stride] */
  uint64_t residual_row_stride; /* elements, 0 = N */
  uint64_t reserved[1];
} ullm_linear_forward_desc_t;

typedef struct ullm_linear_act_quant_desc_t {
  uint32_t struct_size;
  uint32_t abi_version;
  uint64_t m;
  uint64_t k;
  const void *x;         /* device bf16 [M][x_row_stride] */
  uint64_t x_row_stride; /* elements, 0 = K */
  void *xq;              /* device u8 E4M3FN [M][K] */
  float *x_scales;       /* device f32 [M] */
  void *stream;
  uint64_t reserved[4];
} ullm_linear_act_quant_desc_t;

/* Fused add + per-token quantization: the activations quantized are
 * sum = bf16(a + b) (the fp32 sum of each pair of bf16 elements, rounded to
 * nearest even), optionally also written out.  128 bytes. */
typedef struct ullm_linear_add_act_quant_desc_t {
  uint32_t struct_size;
  uint32_t abi_version;
  uint64_t m;
  uint64_t k;
  const void *a;           /* device bf16 [M][a_row_stride] */
  uint64_t a_row_stride;   /* elements, 0 = K */
  const void *b;           /* device bf16 [M][b_row_stride] */
  uint64_t b_row_stride;   /* elements, 0 = K */
  void *sum;               /* device bf16 [M][sum_row_stride], or null (not
                              written); may be a or b itself, same stride;
                              any other overlap of the buffers is undefined */
  uint64_t sum_row_stride; /* elements, 0 = K */
  void *xq;                /* device u8 E4M3FN [M][K] */
  float *x_scales;         /* device f32 [M] */
  void *stream;
  uint64_t reserved[4];
} ullm_linear_add_act_quant_desc_t;

typedef struct ullm_linear_weight_export_desc_t {
  uint32_t struct_size;
  uint32_t abi_version;
  uint32_t memory; /* ULLM_MEMORY_* of the destination buffers */
  uint32_t reserved0;
  void *values; /* canonical layout of the weight's encoding */
  void *scales;
  void *zeros; /* AQ4 only */
  void *stream;
  uint64_t reserved[4];
} ullm_linear_weight_export_desc_t;

/* Kernel families reported by ullm_linear_forward_plan. */
#define ULLM_LINEAR_KERNEL_GEMV UINT32_C(1)        /* decode, bf16 activations */
#define ULLM_LINEAR_KERNEL_GEMM_DIRECT UINT32_C(2) /* FP8 GEMM, operands from L2 */
#define ULLM_LINEAR_KERNEL_GEMM_LDS UINT32_C(3)    /* FP8 GEMM, LDS-pipelined */

/* GEMV kernel variants reported by ullm_linear_forward_plan. */
#define ULLM_LINEAR_GEMV_SINGLE UINT32_C(1)  /* one stripe per workgroup, x from L2 */
#define ULLM_LINEAR_GEMV_SINGLE_LDS UINT32_C(2) /* one stripe per workgroup, x in LDS */
#define ULLM_LINEAR_GEMV_MULTI_STRIPE UINT32_C(3) /* x in LDS, a run of stripes */
#define ULLM_LINEAR_GEMV_REGISTER_STAGED UINT32_C(4) /* x in registers, stripe groups */
#define ULLM_LINEAR_GEMV_SPLIT_K UINT32_C(5) /* register-staged, K split over workgroups */

/* The launch a forward call with a given descriptor makes (diagnostics: the
 * parity tests use it to prove which kernel configuration they cover). */
typedef struct ullm_linear_plan_t {
  uint32_t struct_size;
  uint32_t abi_version;
  uint32_t kernel;  /* ULLM_LINEAR_KERNEL_* (0 when M = 0: nothing runs) */
  uint32_t block_m; /* GEMM: rows x columns of one output tile */
  uint32_t block_n;
  uint32_t tiles;   /* GEMM: output tiles */
  uint32_t grid;    /* GEMM: workgroups; grid < tiles = persistent grid */
  uint32_t split_k; /* K parts per GEMV stripe group or GEMM tile (1 = no split) */
  uint32_t gemv_variant; /* GEMV: ULLM_LINEAR_GEMV_* (0 otherwise) */
  uint32_t gemv_waves;   /* GEMV: waves per workgroup */
  uint32_t gemv_stripes; /* GEMV: stripes sharing one activation load */
  uint32_t gemv_row_classes; /* GEMV: activation row classes per MFMA (1 = none) */
  uint64_t reserved[2];
} ullm_linear_plan_t;

#ifdef __cplusplus
extern "C" {
#endif

/* Create a device-resident weight.  SOURCE_F32 quantizes on the GPU with the
 * encoding's recipe; SOURCE_ENCODED uploads canonical encoded bytes.  Either
 * way the weight is repacked into the device tile layout the kernels stream.
 * Blocks until the weight is ready. */
ULLM_HIP_API ullm_status_t ullm_linear_weight_create(
    const ullm_linear_weight_desc_t *desc, ullm_linear_weight_t **weight,
    ullm_error_sink_t *error_sink);

/* Destroy and null *weight.  Waits for the device to finish using it. */
ULLM_HIP_API ullm_status_t ullm_linear_weight_destroy(
    ullm_linear_weight_t **weight, ullm_error_sink_t *error_sink);

ULLM_HIP_API ullm_status_t ullm_linear_weight_query(
    const ullm_linear_weight_t *weight, ullm_linear_weight_info_t *info,
    ullm_error_sink_t *error_sink);

/* Write the canonical encoded bytes back out (exact inverse of the repack). */
ULLM_HIP_API ullm_status_t ullm_linear_weight_export(
    const ullm_linear_weight_t *weight,
    const ullm_linear_weight_export_desc_t *desc,
    ullm_error_sink_t *error_sink);

/* Parity/debug: dequantized weights as f32 [N][K] into device memory, with
 * the exact operation order of the encoding's definition.  Stream-ordered. */
ULLM_HIP_API ullm_status_t ullm_linear_weight_dequantize(
    const ullm_linear_weight_t *weight, float *out, void *stream,
    ullm_error_sink_t *error_sink);

/* Y = alpha * X * W^T, then the descriptor's epilogue.  Stream-ordered.
 * A gated-pair weight requires ULLM_LINEAR_EPILOGUE_SILU_MUL (its Y has N / 2
 * columns); SILU_MUL requires a gated-pair weight. */
ULLM_HIP_API ullm_status_t ullm_linear_forward(
    const ullm_linear_forward_desc_t *desc, ullm_error_sink_t *error_sink);

/* Bytes of workspace ullm_linear_forward needs for this descriptor: for the
 * prefill GEMM the split-K counters and partial sums (grids of few output
 * tiles split K over workgroups) and, for bf16 activations, their per-token
 * quantization; for a decode call that splits K (9 <= M <= 32, few output
 * rows, long K) its split-K scratch; 0 when the call needs none. */
ULLM_HIP_API ullm_status_t ullm_linear_workspace_size(
    const ullm_linear_forward_desc_t *desc, uint64_t *bytes,
    ullm_error_sink_t *error_sink);

/* The kernel family and launch geometry ullm_linear_forward would use for
 * this descriptor on the weight's device.  Launches nothing.  No counterpart
 * in the reference: a diagnostic for parity tests and tuning reports. */
ULLM_HIP_API ullm_status_t ullm_linear_forward_plan(
    const ullm_linear_forward_desc_t *desc, ullm_linear_plan_t *plan,
    ullm_error_sink_t *error_sink);

/* ullm_linear_forward without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same descriptor, validation and result as ullm_linear_forward, except that
 * desc->workspace must be null: all scratch comes from a fixed per-device
 * array of 32 MiB held by the library for the life of the process (64 KiB of
 * split-K counters plus 32 MiB - 64 KiB for split-K partials and the prefill
 * path's quantized activations, M*K + 4*M bytes each rounded up to 256).
 * Calls needing more are refused with ULLM_STATUS_UNSUPPORTED.  All calls on
 * one device share that array: calls that overlap in time on one device
 * (different streams or threads) race and must be ordered by the caller. */
ULLM_HIP_API ullm_status_t ullm_linear_forward_noalloc(
    const ullm_linear_forward_desc_t *desc, ullm_error_sink_t *error_sink);

/* Free every library-owned workspace of `device` (the buffers forward calls
 * made with a null workspace, including those retired when a larger one
 * replaced them), after waiting for the device.  HIP graphs captured with
 * those buffers must not be replayed afterwards; later calls allocate anew.
 * No counterpart in the reference. */
ULLM_HIP_API ullm_status_t ullm_linear_release_workspaces(
    int32_t device, ullm_error_sink_t *error_sink);

/* Per-token E4M3 quantization of bf16 activations.  Stream-ordered. */
ULLM_HIP_API ullm_status_t ullm_linear_quantize_activations(
    const ullm_linear_act_quant_desc_t *desc, ullm_error_sink_t *error_sink);

/* Per-token E4M3 quantization of a + b (bf16), the add that precedes a
 * linear layer (a residual add) fused into the quantization pass: the sum
 * is read once, and written only when `sum` is set.  xq and x_scales equal
 * those of ullm_linear_quantize_activations on the rounded sum.  Replaces
 * the reference's elementwise Add (crates/ullm-core/src/op.rs:90-95: two
 * inputs and the output of one shape and dtype) followed by the Matmul's
 * activation quantization; the reference defines no numerics for Add.
 * Stream-ordered. */
ULLM_HIP_API ullm_status_t ullm_linear_add_quantize_activations(
    const ullm_linear_add_act_quant_desc_t *desc, ullm_error_sink_t *error_sink);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* ULLM_LINEAR_H */
