/*
 * ullm_oracle.c -- CPU restatement of the quantized linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY (see ullm_oracle.h).  Built with
 * -ffp-contract=off so that every multiply and add rounds separately, as the
 * definitions in the header state.
 *
 * Reference anchors: the reference defines the storage types only
 * (crates/ullm-core/src/dtype.rs:10 F8E4M3Fn, :7 Bf16, :8 F16) and the Matmul
 * shape contract A[M,K] x B[K,N] (crates/ullm-core/src/op.rs:97-113).  The
 * quantization recipes restate BASELINE configurations #1-#4; there is no
 * reference implementation to follow line by line.
 */
#include "ullm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------------- */
/* Generic binary minifloat rounding, from the definition of the formats:  */
/* a finite value is sign * 2^E * (1 + f/2^mbits) for E >= emin, or        */
/* sign * 2^emin * (f/2^mbits) below it.  Rounding to nearest even on the  */
/* grid of spacing 2^(E - mbits) is one nearbyint() in double, which is    */
/* exact because every float is a double and the grid spacing is a power   */
/* of two.                                                                 */
/* ---------------------------------------------------------------------- */

static double mf_round(double a, int mbits, int emin) {
  int e;
  (void)frexp(a, &e); /* a in [2^(e-1), 2^e) */
  int E = e - 1;
  if (E < emin) {
    E = emin;
  }
  const double quantum = ldexp(1.0, E - mbits);
  return nearbyint(a / quantum) * quantum;
}

/* Encode a rounded, representable, positive magnitude r into exponent and
 * mantissa fields. */
static uint32_t mf_fields(double r, int mbits, int emin) {
  const int bias = 1 - emin;
  if (r == 0.0) {
    return 0U;
  }
  if (r < ldexp(1.0, emin)) { /* subnormal */
    return (uint32_t)(r / ldexp(1.0, emin - mbits));
  }
  int e;
  (void)frexp(r, &e);
  const int E = e - 1;
  const uint32_t mant =
      (uint32_t)(r / ldexp(1.0, E - mbits)) - (1U << (unsigned)mbits);
  return ((uint32_t)(E + bias) << (unsigned)mbits) | mant;
}

static double mf_decode(uint32_t fields, int mbits, int emin) {
  const int bias = 1 - emin;
  const uint32_t mant = fields & ((1U << (unsigned)mbits) - 1U);
  const int ef = (int)(fields >> (unsigned)mbits);
  if (ef == 0) {
    return ldexp((double)mant, emin - mbits);
  }
  return ldexp((double)((1U << (unsigned)mbits) + mant), ef - bias - mbits);
}

static uint32_t f32_bits(float x) {
  uint32_t b;
  memcpy(&b, &x, sizeof b);
  return b;
}

/* E4M3FN: mbits 3, emin -6 (bias 7), max 448 = 1.75 * 2^8, NaN 0x7F. */
uint8_t orc_e4m3_from_f32(float x) {
  const uint8_t sign = (f32_bits(x) >> 31) ? 0x80U : 0x00U;
  if (isnan(x)) {
    return (uint8_t)(sign | 0x7FU);
  }
  const double a = fabs((double)x);
  if (a >= 448.0) {
    return (uint8_t)(sign | 0x7EU);
  }
  if (a == 0.0) {
    return sign;
  }
  const double r = mf_round(a, 3, -6); /* r <= 448 because 448 is on the grid */
  return (uint8_t)(sign | mf_fields(r, 3, -6));
}

float orc_e4m3_to_f32(uint8_t code) {
  const double sign = (code & 0x80U) ? -1.0 : 1.0;
  if ((code & 0x7FU) == 0x7FU) {
    return NAN;
  }
  return (float)(sign * mf_decode(code & 0x7FU, 3, -6));
}

/* bf16: mbits 7, emin -126, overflow to inf at 2^128. */
uint16_t orc_bf16_from_f32(float x) {
  const uint16_t sign = (f32_bits(x) >> 31) ? 0x8000U : 0U;
  if (isnan(x)) {
    return (uint16_t)(sign | 0x7FC0U);
  }
  const double a = fabs((double)x);
  if (isinf(a)) {
    return (uint16_t)(sign | 0x7F80U);
  }
  if (a == 0.0) {
    return sign;
  }
  const double r = mf_round(a, 7, -126);
  if (r >= ldexp(1.0, 128)) {
    return (uint16_t)(sign | 0x7F80U);
  }
  return (uint16_t)(sign | mf_fields(r, 7, -126));
}

float orc_bf16_to_f32(uint16_t bits) {
  const uint32_t b = (uint32_t)bits << 16U;
  float f;
  memcpy(&f, &b, sizeof f);
  return f;
}

/* f16: mbits 10, emin -14, overflow to inf at 2^16. */
uint16_t orc_f16_from_f32(float x) {
  const uint16_t sign = (f32_bits(x) >> 31) ? 0x8000U : 0U;
  if (isnan(x)) {
    return (uint16_t)(sign | 0x7E00U);
  }
  const double a = fabs((double)x);
  if (isinf(a)) {
    return (uint16_t)(sign | 0x7C00U);
  }
  if (a == 0.0) {
    return sign;
  }
  const double r = mf_round(a, 10, -14);
  if (r >= 65536.0) {
    return (uint16_t)(sign | 0x7C00U);
  }
  return (uint16_t)(sign | mf_fields(r, 10, -14));
}

float orc_f16_to_f32(uint16_t bits) {
  const double sign = (bits & 0x8000U) ? -1.0 : 1.0;
  const uint32_t mag = bits & 0x7FFFU;
  if ((mag >> 10) == 0x1FU) {
    return (mag & 0x3FFU) ? NAN : (float)(sign * INFINITY);
  }
  return (float)(sign * mf_decode(mag, 10, -14));
}

void orc_e4m3_from_f32_n(const float *x, uint8_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    out[i] = orc_e4m3_from_f32(x[i]);
  }
}

void orc_bf16_from_f32_n(const float *x, uint16_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    out[i] = orc_bf16_from_f32(x[i]);
  }
}

void orc_f16_from_f32_n(const float *x, uint16_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    out[i] = orc_f16_from_f32(x[i]);
  }
}

/* ---------------------------------------------------------------------- */
/* Weight quantization                                                     */
/* ---------------------------------------------------------------------- */

void orc_fp8_quantize_rows(const float *w, int64_t n, int64_t k, uint8_t *q,
                           float *s) {
  for (int64_t r = 0; r < n; ++r) {
    const float *row = w + r * k;
    float amax = 0.0f;
    for (int64_t c = 0; c < k; ++c) {
      const float a = fabsf(row[c]);
      if (a > amax) {
        amax = a;
      }
    }
    const float scale = amax / 448.0f;
    s[r] = scale;
    for (int64_t c = 0; c < k; ++c) {
      q[r * k + c] = scale == 0.0f ? (uint8_t)0 : orc_e4m3_from_f32(row[c] / scale);
    }
  }
}

void orc_fp8_dequantize(const uint8_t *q, const float *s, int64_t n, int64_t k,
                        float *out) {
  for (int64_t r = 0; r < n; ++r) {
    for (int64_t c = 0; c < k; ++c) {
      out[r * k + c] = orc_e4m3_to_f32(q[r * k + c]) * s[r];
    }
  }
}

void orc_aq4_quantize(const float *w, int64_t n, int64_t k, uint32_t *packed,
                      uint16_t *scales, uint16_t *zeros) {
  const int64_t groups = k / 128;
  memset(packed, 0, (size_t)(n * (k / 8)) * sizeof(uint32_t));
  for (int64_t r = 0; r < n; ++r) {
    for (int64_t g = 0; g < groups; ++g) {
      const float *v = w + r * k + g * 128;
      float lo = v[0];
      float hi = v[0];
      for (int i = 1; i < 128; ++i) {
        lo = v[i] < lo ? v[i] : lo;
        hi = v[i] > hi ? v[i] : hi;
      }
      uint16_t s16 = orc_f16_from_f32((hi - lo) / 15.0f);
      uint16_t z16 = 0;
      if (orc_f16_to_f32(s16) != 0.0f) {
        z16 = orc_f16_from_f32(-lo / orc_f16_to_f32(s16));
      }
      if (orc_f16_to_f32(s16) == 0.0f || !isfinite(orc_f16_to_f32(z16))) {
        s16 = 0x3C00U; /* 1.0 */
        z16 = orc_f16_from_f32(-lo);
      }
      scales[r * groups + g] = s16;
      zeros[r * groups + g] = z16;
      const float sf = orc_f16_to_f32(s16);
      const float zf = orc_f16_to_f32(z16);
      for (int i = 0; i < 128; ++i) {
        const float t = v[i] / sf;
        float u = nearbyintf(t + zf);
        u = u < 0.0f ? 0.0f : (u > 15.0f ? 15.0f : u);
        const uint32_t qv = (uint32_t)u;
        const int64_t kk = g * 128 + i;
        packed[r * (k / 8) + kk / 8] |= qv << (4U * (uint32_t)(kk % 8));
      }
    }
  }
}

static inline uint32_t aq4_code(const uint32_t *packed, int64_t k, int64_t r,
                                int64_t c) {
  return (packed[r * (k / 8) + c / 8] >> (4U * (uint32_t)(c % 8))) & 0xFU;
}

void orc_aq4_dequantize(const uint32_t *packed, const uint16_t *scales,
                        const uint16_t *zeros, int64_t n, int64_t k,
                        float *out) {
  const int64_t groups = k / 128;
  for (int64_t r = 0; r < n; ++r) {
    for (int64_t c = 0; c < k; ++c) {
      const float sf = orc_f16_to_f32(scales[r * groups + c / 128]);
      const float zf = orc_f16_to_f32(zeros[r * groups + c / 128]);
      out[r * k + c] = ((float)aq4_code(packed, k, r, c) - zf) * sf;
    }
  }
}

/* ---------------------------------------------------------------------- */
/* Contractions                                                            */
/* ---------------------------------------------------------------------- */

static void set_threads(int threads) {
#ifdef _OPENMP
  if (threads > 0) {
    omp_set_num_threads(threads);
  }
#else
  (void)threads;
#endif
}

int orc_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

static float *bf16_rows_to_f32(int64_t m, int64_t k, const uint16_t *x,
                               int64_t ldx) {
  float *xf = (float *)malloc((size_t)(m * k) * sizeof(float));
  for (int64_t i = 0; i < m; ++i) {
    for (int64_t c = 0; c < k; ++c) {
      xf[i * k + c] = orc_bf16_to_f32(x[i * ldx + c]);
    }
  }
  return xf;
}

void orc_fp8_gemv(int64_t m, int64_t n, int64_t k, const uint16_t *x,
                  int64_t ldx, const uint8_t *q, const float *s, float alpha,
                  float *y32, double *y64, int threads) {
  float lut[256];
  for (int i = 0; i < 256; ++i) {
    lut[i] = orc_e4m3_to_f32((uint8_t)i);
  }
  float *xf = bf16_rows_to_f32(m, k, x, ldx);
  set_threads(threads);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < n; ++r) {
    const uint8_t *row = q + r * k;
    for (int64_t i = 0; i < m; ++i) {
      const float *xr = xf + i * k;
      if (y32 != NULL) {
        float acc = 0.0f;
        for (int64_t c = 0; c < k; ++c) {
          acc += lut[row[c]] * xr[c];
        }
        y32[i * n + r] = alpha * (s[r] * acc);
      }
      if (y64 != NULL) {
        double acc = 0.0;
        for (int64_t c = 0; c < k; ++c) {
          acc += (double)lut[row[c]] * (double)xr[c];
        }
        y64[i * n + r] = (double)alpha * ((double)s[r] * acc);
      }
    }
  }
  free(xf);
}

void orc_aq4_gemv(int64_t m, int64_t n, int64_t k, const uint16_t *x,
                  int64_t ldx, const uint32_t *packed, const uint16_t *scales,
                  const uint16_t *zeros, float alpha, float *y32, double *y64,
                  int threads) {
  float *xf = bf16_rows_to_f32(m, k, x, ldx);
  const int64_t groups = k / 128;
  set_threads(threads);
#pragma omp parallel
  {
    float *wd = (float *)malloc((size_t)k * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t r = 0; r < n; ++r) {
      for (int64_t c = 0; c < k; ++c) {
        const float sf = orc_f16_to_f32(scales[r * groups + c / 128]);
        const float zf = orc_f16_to_f32(zeros[r * groups + c / 128]);
        wd[c] = ((float)aq4_code(packed, k, r, c) - zf) * sf;
      }
      for (int64_t i = 0; i < m; ++i) {
        const float *xr = xf + i * k;
        if (y32 != NULL) {
          float acc = 0.0f;
          for (int64_t c = 0; c < k; ++c) {
            acc += wd[c] * xr[c];
          }
          y32[i * n + r] = alpha * acc;
        }
        if (y64 != NULL) {
          double acc = 0.0;
          for (int64_t c = 0; c < k; ++c) {
            acc += (double)wd[c] * (double)xr[c];
          }
          y64[i * n + r] = (double)alpha * acc;
        }
      }
    }
    free(wd);
  }
  free(xf);
}

void orc_bf16_add(int64_t n, const uint16_t *a, const uint16_t *b, uint16_t *out) {
  for (int64_t i = 0; i < n; ++i) {
    out[i] = orc_bf16_from_f32(orc_bf16_to_f32(a[i]) + orc_bf16_to_f32(b[i]));
  }
}

void orc_act_quantize(int64_t m, int64_t k, const uint16_t *x, int64_t ldx,
                      uint8_t *xq, float *xs) {
  for (int64_t i = 0; i < m; ++i) {
    float amax = 0.0f;
    for (int64_t c = 0; c < k; ++c) {
      const float a = fabsf(orc_bf16_to_f32(x[i * ldx + c]));
      amax = a > amax ? a : amax;
    }
    const float scale = amax / 448.0f;
    xs[i] = scale;
    for (int64_t c = 0; c < k; ++c) {
      xq[i * k + c] = scale == 0.0f
                          ? (uint8_t)0
                          : orc_e4m3_from_f32(orc_bf16_to_f32(x[i * ldx + c]) / scale);
    }
  }
}

void orc_fp8_gemm(int64_t m, int64_t n, int64_t k, const uint8_t *xq,
                  const float *xs, const uint8_t *q, const float *s,
                  float alpha, float *y32, double *y64, int threads) {
  float lut[256];
  for (int i = 0; i < 256; ++i) {
    lut[i] = orc_e4m3_to_f32((uint8_t)i);
  }
  set_threads(threads);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < n; ++r) {
    const uint8_t *row = q + r * k;
    for (int64_t i = 0; i < m; ++i) {
      const uint8_t *xr = xq + i * k;
      if (y32 != NULL) {
        float acc = 0.0f;
        for (int64_t c = 0; c < k; ++c) {
          acc += lut[row[c]] * lut[xr[c]];
        }
        y32[i * n + r] = alpha * ((xs[i] * s[r]) * acc);
      }
      if (y64 != NULL) {
        double acc = 0.0;
        for (int64_t c = 0; c < k; ++c) {
          acc += (double)lut[row[c]] * (double)lut[xr[c]];
        }
        y64[i * n + r] = (double)alpha * ((double)xs[i] * (double)s[r] * acc);
      }
    }
  }
}

/* SiLU-gate epilogue: gate columns [0, f), up columns [f, 2f) of each row. */
void orc_silu_mul(int64_t m, int64_t f, const float *gu, float *out) {
  for (int64_t i = 0; i < m; ++i) {
    for (int64_t j = 0; j < f; ++j) {
      const float g = gu[i * 2 * f + j];
      const float u = gu[i * 2 * f + f + j];
      const float silu = g / (1.0f + expf(-g));
      out[i * f + j] = silu * u;
    }
  }
}
