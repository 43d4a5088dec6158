/* archive_check.c -- a C program linked against the CMake target's static
 * archive (libullm_hip_stub.a) the way the reference's ullm-hip-sys links it
 * (static archive + amdhip64 + stdc++).  On a gfx950 device it creates an
 * FP8 and an AQ4 weight from host f32 values, runs a forward at M = 2, and
 * checks the bf16 outputs against dot products of the library's own
 * dequantized weights (ullm_linear_weight_dequantize) with the same bf16
 * activations, in double precision, within 1e-2 x RMS.  This checks that the
 * archive's kernels are registered and run when linked statically; the
 * numerics themselves are pinned against the oracle by the Python suite.
 * Prints "ok" and exits 0 on success; "skip" (exit 0) without a gfx950. */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ullm/linear.h"

#define M 2
#define N 48
#define K 256

static uint32_t rng = 12345u;
static float uniform(void) { /* xorshift32 in [-1, 1) */
  rng ^= rng << 13;
  rng ^= rng >> 17;
  rng ^= rng << 5;
  return (float)((double)rng / 2147483648.0 - 1.0);
}

static uint16_t bf16_bits(float f) { /* round to nearest even (finite values) */
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float bf16_value(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

#define CHECK_HIP(e)                                                  \
  do {                                                                \
    hipError_t err_ = (e);                                            \
    if (err_ != hipSuccess) {                                         \
      printf("FAIL %s:%d %s\n", __FILE__, __LINE__, hipGetErrorName(err_)); \
      return 1;                                                       \
    }                                                                 \
  } while (0)
#define CHECK_ST(e)                                                   \
  do {                                                                \
    ullm_status_t st_ = (e);                                          \
    if (st_ != ULLM_STATUS_OK) {                                      \
      printf("FAIL %s:%d status %u: %s\n", __FILE__, __LINE__, st_, msg); \
      return 1;                                                       \
    }                                                                 \
  } while (0)

static char msg[256];

static int run(uint32_t encoding, const float *w, const uint16_t *xh, void *dx,
               void *dy, float *dwd) {
  ullm_error_sink_t sink = ULLM_ERROR_SINK_INIT(msg);
  ullm_linear_weight_desc_t wd;
  memset(&wd, 0, sizeof wd);
  wd.struct_size = sizeof wd;
  wd.abi_version = ULLM_HIP_ABI_VERSION;
  wd.encoding = encoding;
  wd.source = ULLM_LINEAR_SOURCE_F32;
  wd.n = N;
  wd.k = K;
  wd.memory = ULLM_MEMORY_HOST;
  wd.values = w;
  ullm_linear_weight_t *weight = NULL;
  CHECK_ST(ullm_linear_weight_create(&wd, &weight, &sink));

  ullm_linear_forward_desc_t fd;
  memset(&fd, 0, sizeof fd);
  fd.struct_size = sizeof fd;
  fd.abi_version = ULLM_HIP_ABI_VERSION;
  fd.weight = weight;
  fd.m = M;
  fd.x = dx;
  fd.y = dy;
  fd.x_dtype = ULLM_LINEAR_DTYPE_BF16;
  fd.y_dtype = ULLM_LINEAR_DTYPE_BF16;
  fd.activation_mode = ULLM_LINEAR_ACT_EXACT;
  fd.alpha = 1.0f;
  CHECK_ST(ullm_linear_forward(&fd, &sink));
  CHECK_ST(ullm_linear_weight_dequantize(weight, dwd, NULL, &sink));
  CHECK_HIP(hipDeviceSynchronize());

  static uint16_t y[M * N];
  static float wdq[N * K];
  CHECK_HIP(hipMemcpy(y, dy, sizeof y, hipMemcpyDeviceToHost));
  CHECK_HIP(hipMemcpy(wdq, dwd, sizeof wdq, hipMemcpyDeviceToHost));
  double ref[M * N], ss = 0.0, worst = 0.0;
  for (int m = 0; m < M; ++m) {
    for (int n = 0; n < N; ++n) {
      double acc = 0.0;
      for (int k = 0; k < K; ++k) {
        acc += (double)wdq[n * K + k] * (double)bf16_value(xh[m * K + k]);
      }
      ref[m * N + n] = acc;
      ss += acc * acc;
    }
  }
  const double rms = sqrt(ss / (M * N));
  for (int i = 0; i < M * N; ++i) {
    const double d = fabs((double)bf16_value(y[i]) - ref[i]);
    /* the reference itself rounds to bf16: half an ulp of |ref| on top */
    const double slack = fabs(ref[i]) * 0.00390625 / 2.0;
    if (d - slack > worst) {
      worst = d - slack;
    }
  }
  CHECK_ST(ullm_linear_weight_destroy(&weight, &sink));
  if (!(rms > 0.0) || worst > 1e-2 * rms) {
    printf("FAIL encoding %u: max |dy| %g against 1e-2 x RMS %g\n", encoding, worst, rms);
    return 1;
  }
  return 0;
}

int main(void) {
  ullm_error_sink_t sink = ULLM_ERROR_SINK_INIT(msg);
  ullm_backend_probe_result_t probe;
  memset(&probe, 0, sizeof probe);
  probe.struct_size = sizeof probe;
  probe.abi_version = ULLM_HIP_ABI_VERSION;
  if (ullm_backend_probe(ULLM_BACKEND_HIP, &probe, &sink) != ULLM_STATUS_OK ||
      !probe.available) {
    printf("skip: %s\n", msg);
    return 0;
  }
  static float w[N * K];
  static uint16_t xh[M * K];
  for (int i = 0; i < N * K; ++i) {
    w[i] = 0.02f * uniform();
  }
  for (int i = 0; i < M * K; ++i) {
    xh[i] = bf16_bits(uniform());
  }
  void *dx = NULL, *dy = NULL;
  float *dwd = NULL;
  CHECK_HIP(hipMalloc(&dx, sizeof xh));
  CHECK_HIP(hipMalloc(&dy, sizeof(uint16_t) * M * N));
  CHECK_HIP(hipMalloc((void **)&dwd, sizeof(float) * N * K));
  CHECK_HIP(hipMemcpy(dx, xh, sizeof xh, hipMemcpyHostToDevice));
  if (run(ULLM_LINEAR_ENCODING_FP8_E4M3_ROW, w, xh, dx, dy, dwd) != 0 ||
      run(ULLM_LINEAR_ENCODING_AQ4_G128, w, xh, dx, dy, dwd) != 0) {
    return 1;
  }
  CHECK_HIP(hipFree(dx));
  CHECK_HIP(hipFree(dy));
  CHECK_HIP(hipFree(dwd));
  printf("ok\n");
  return 0;
}
