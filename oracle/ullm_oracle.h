/*
 * ullm_oracle.h -- CPU restatement of the quantized linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP
 * kernels in ullm-project_amd/src are compared against.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product library never links or calls it.
 *
 * The reference (jyohukuchan/uLLM-project) has no numerical implementation of
 * this path: it stops at the type vocabulary (crates/ullm-core/src/dtype.rs:6-16
 * DType::F8E4M3Fn, dtype.rs:55-66 Encoding) and a shape-only Matmul descriptor
 * (crates/ullm-core/src/op.rs:97-113).  Every numeric contract below is
 * therefore this build's definition of the BASELINE configurations, written
 * from the mathematics of each format:
 *
 *   e4m3fn   OCP FP8 E4M3 "fn": bias 7, 3 mantissa bits, max finite 448, no
 *            infinities, NaN = S.1111.111.  Encoding rounds to nearest even and
 *            saturates every |x| >= 448 (including +-inf) to +-448.
 *   bf16     IEEE-style binary16 with 8 exponent bits, RNE, overflow -> inf.
 *   f16      IEEE binary16, RNE, subnormals kept, overflow -> inf.
 *
 *   FP8 row weights   s_n = max_k |W[n,k]| / 448 (fp32 division);
 *                     Q[n,k] = e4m3(W[n,k] / s_n); s_n == 0 -> Q = 0.
 *                     dequant: Wd = e4m3_to_f32(Q) * s_n (one fp32 multiply).
 *   AQ4 g128 weights  per row n and group g of 128 consecutive k:
 *                     lo = min, hi = max (fp32);
 *                     s16 = f16((hi - lo) / 15.0f);  z16 = f16(-lo / float(s16));
 *                     degenerate (s16 == 0 or z16 not finite): s16 = 1, z16 = f16(-lo);
 *                     q = clamp(rint(w / s + z), 0, 15)   (fp32 div, fp32 add, RNE);
 *                     dequant: Wd = (float(q) - z) * s    (two fp32 ops, no FMA).
 *                     Packed: u32 P[n][k/8], nibble j of word w holds k = 8w + j,
 *                     low nibble first; S, Z are f16 [n][k/128].
 *   matvec/GEMV       Y32[m,n] = alpha * (s_n * sum_k e4m3(Q[n,k]) * x[m,k]),
 *                     fp32 accumulation in increasing k.  AQ4 uses Wd.
 *   act quant         a_m = max_k |x[m,k]| / 448; XA = e4m3(x / a_m); a_m == 0 -> XA = 0.
 *   FP8 GEMM          Y32[m,n] = alpha * ((a_m * s_n) * sum_k e4m3(XA) * e4m3(Q)).
 *   SiLU-gate epilogue  for a fused gate/up product Y32[m][2F] (gate columns
 *                     0..F-1, up columns F..2F-1, alpha already applied):
 *                     out[m,j] = silu(Y32[m,j]) * Y32[m,F+j],
 *                     silu(v) = v / (1 + expf(-v))  (fp32, libm expf).
 *                     No reference file defines it: the survey lists the fused
 *                     SiLU-gate epilogue as the path's next step, and this is
 *                     the standard SwiGLU gate (x * sigmoid(x)).
 *   residual epilogue Y32 + R, one fp32 add per element.
 *
 * All functions take row strides in elements where a caller may hand a view.
 */
#ifndef ULLM_ORACLE_H
#define ULLM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* scalar formats */
uint8_t orc_e4m3_from_f32(float x);
float orc_e4m3_to_f32(uint8_t code);
uint16_t orc_bf16_from_f32(float x);
float orc_bf16_to_f32(uint16_t bits);
uint16_t orc_f16_from_f32(float x);
float orc_f16_to_f32(uint16_t bits);

/* vector conversions (for tests that sweep many values) */
void orc_e4m3_from_f32_n(const float *x, uint8_t *out, int64_t n);
void orc_bf16_from_f32_n(const float *x, uint16_t *out, int64_t n);
void orc_f16_from_f32_n(const float *x, uint16_t *out, int64_t n);

/* FP8-E4M3 per-row weights */
void orc_fp8_quantize_rows(const float *w, int64_t n, int64_t k, uint8_t *q,
                           float *s);
void orc_fp8_dequantize(const uint8_t *q, const float *s, int64_t n, int64_t k,
                        float *out);

/* AQ4 g128 weights; k must be a multiple of 128 */
void orc_aq4_quantize(const float *w, int64_t n, int64_t k, uint32_t *packed,
                      uint16_t *scales, uint16_t *zeros);
void orc_aq4_dequantize(const uint32_t *packed, const uint16_t *scales,
                        const uint16_t *zeros, int64_t n, int64_t k,
                        float *out);

/* bf16-activation matvec / small-M GEMV.  y32 is fp32 [m][n] (before the
 * bf16 output rounding), y64 the same sum accumulated in double.  Either
 * output may be NULL.  threads <= 0 uses the OpenMP default. */
void orc_fp8_gemv(int64_t m, int64_t n, int64_t k, const uint16_t *x,
                  int64_t ldx, const uint8_t *q, const float *s, float alpha,
                  float *y32, double *y64, int threads);
void orc_aq4_gemv(int64_t m, int64_t n, int64_t k, const uint16_t *x,
                  int64_t ldx, const uint32_t *packed, const uint16_t *scales,
                  const uint16_t *zeros, float alpha, float *y32, double *y64,
                  int threads);

/* Elementwise bf16 add (the Add that precedes a linear layer, whose shape
 * contract is the reference's crates/ullm-core/src/op.rs:90-95; the reference
 * defines no numerics for it): out = bf16(f32(a) + f32(b)), the fp32 sum
 * rounded to nearest even.  Feeds the fused add + quantization. */
void orc_bf16_add(int64_t n, const uint16_t *a, const uint16_t *b, uint16_t *out);

/* per-token activation quantization and the FP8 x FP8 GEMM */
void orc_act_quantize(int64_t m, int64_t k, const uint16_t *x, int64_t ldx,
                      uint8_t *xq, float *xs);
void orc_fp8_gemm(int64_t m, int64_t n, int64_t k, const uint8_t *xq,
                  const float *xs, const uint8_t *q, const float *s,
                  float alpha, float *y32, double *y64, int threads);

/* epilogues on an fp32 product (see the definitions above) */
void orc_silu_mul(int64_t m, int64_t f, const float *gu, float *out);

/* number of OpenMP threads the library would use for threads <= 0 */
int orc_max_threads(void);

#ifdef __cplusplus
}
#endif

#endif /* ULLM_ORACLE_H */
