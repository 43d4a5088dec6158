/* act_quant_division_check.c -- exhaustive check of the per-token activation
 * quantizer's division (ullm-project_amd/src/weights.hip,
 * act_quant_vec_kernel): for a row scale a = max|x| / 448 >= 2^-100 the
 * kernel computes x / a as q0 = x * r, q = fma(fma(-q0, a, x), r, q0) with
 * r = 1 / a (keeping q0 when it is zero), and divides otherwise.  For every
 * finite positive bf16 row maximum and every bf16 x with |x| <= it, the
 * E4M3 code of that quotient must equal the code of the correctly rounded
 * x / a (the oracle's encode, oracle/ullm_oracle.c).  Prints the counts;
 * exits 1 on any code mismatch.  Built and run by
 * tests/test_act_quant_division.py. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "ullm_oracle.h"

static float f_of(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint32_t u_of(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

int main(void) {
  long long pairs = 0, fp32_diff = 0, code_diff = 0;
#pragma omp parallel for reduction(+ : pairs, fp32_diff, code_diff) schedule(dynamic)
  for (uint32_t am = 1; am < 0x7f80u; ++am) {
    const float a = f_of(am << 16) / 448.0f;
    if (a == 0.0f) {
      continue;
    }
    const float r = 1.0f / a;
    const int via_rcp = a >= 0x1p-100f;
    for (uint32_t xb = 0; xb < 0x10000u; ++xb) {
      if ((xb & 0x7fffu) > am) {
        continue;
      }
      const float x = f_of(xb << 16);
      const float exact = x / a;
      float q = exact;
      if (via_rcp) {
        const float q0 = x * r;
        const float q1 = fmaf(fmaf(-q0, a, x), r, q0);
        q = q0 == 0.0f ? q0 : q1;
      }
      pairs++;
      fp32_diff += u_of(q) != u_of(exact);
      code_diff += orc_e4m3_from_f32(q) != orc_e4m3_from_f32(exact);
    }
  }
  printf("pairs %lld fp32_diff %lld code_diff %lld\n", pairs, fp32_diff, code_diff);
  return code_diff != 0;
}
