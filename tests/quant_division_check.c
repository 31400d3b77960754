/* Exhaustive check of the INT8 quantizer's division (test infrastructure).
 *
 * The reference quantizes q = clamp(rint(x / s), -127, 127) with s =
 * max(absmax, 1e-8) / 127 and x / s an IEEE fp32 division (model/int8.py:66-67).
 * The gfx950 kernels instead compute q0 = x * (1/s), r = fma(-q0, s, x),
 * q1 = fma(r, 1/s, q0) and round q1 by adding 1.5 * 2^23, reading the low byte.
 * This program runs both over every positive finite bf16 absmax and every bf16
 * x (both signs) with |x| <= absmax, and prints the number of differences.
 *
 * It also checks the three-operation form used where absmax < 2^80: with
 * hi = 1/s and lo = fma(-s, hi, 1) * hi (so that hi + lo is 1/s to about
 * 2^-47 relative; below 2^80 lo is a normal number or zero),
 * q = rint(fma(x, hi, x * lo)). It fails on a few pairs with absmax >= 2^125,
 * where lo is subnormal, hence the bound.
 * Build: gcc -O2 -ffp-contract=off -fopenmp quant_division_check.c -lm */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float bf16_value(uint32_t h) {
  const uint32_t u = h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static int kernel_q(float x, float s, float inv) {
  const float q0 = x * inv;
  const float r = fmaf(-q0, s, x);
  const float q1 = fmaf(r, inv, q0);
  const float t = q1 + 0x1.8p23f;
  uint32_t bits;
  memcpy(&bits, &t, 4);
  return (int)(int8_t)(bits & 0xffu);
}

static int split_q(float x, float hi, float lo) {
  const float p = fmaf(x, hi, x * lo);
  const float t = p + 0x1.8p23f;
  uint32_t bits;
  memcpy(&bits, &t, 4);
  return (int)(int8_t)(bits & 0xffu);
}

static int reference_q(float x, float s) {
  return (int)fminf(fmaxf(rintf(x / s), -127.0f), 127.0f);
}

int main(void) {
  long cases = 0, diffs = 0, plain_diffs = 0, split_cases = 0, split_diffs = 0;
#pragma omp parallel for schedule(dynamic, 64) \
    reduction(+ : cases, diffs, plain_diffs, split_cases, split_diffs)
  for (int a = 1; a < 0x7f80; ++a) {
    const float absmax = bf16_value((uint32_t)a);
    const float s = fmaxf(absmax, 1e-8f) / 127.0f;
    const float inv = 1.0f / s;
    const int split = absmax < 0x1p80f;
    const float lo = fmaf(-s, inv, 1.0f) * inv;
    for (int b = 0; b <= a; ++b) {
      for (int sign = 0; sign < 2; ++sign) {
        const float x = bf16_value((uint32_t)b | ((uint32_t)sign << 15));
        const int want = reference_q(x, s);
        ++cases;
        if (kernel_q(x, s, inv) != want) ++diffs;
        if ((int)rintf(x * inv) != want) ++plain_diffs;
        if (split) {
          ++split_cases;
          if (split_q(x, inv, lo) != want) ++split_diffs;
        }
      }
    }
  }
  printf("cases %ld differences %ld reciprocal-only-differences %ld split-cases %ld split-differences %ld\n",
         cases, diffs, plain_diffs, split_cases, split_diffs);
  return diffs != 0 || split_diffs != 0;
}
