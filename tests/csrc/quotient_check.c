/* Exhaustive CPU check of the quantizer's fast quotient (fp8_common.h:
 * quotient + copysign) against IEEE float division, for every pair of a bf16
 * value x and a bf16 row maximum a >= |x| (finite rows). The per-row scale is
 * max(a, fp32(1e-12)) * fp32(1/448) and r = RN(1/scale), as on the device.
 * x86-64 SSE arithmetic and fmaf are IEEE binary32 with subnormals, which is
 * also what gfx950's v_mul_f32 / v_fma_f32 compute with denormals enabled.
 *
 * Claims checked:
 *   1. the e4m3 code of the fast quotient equals the code of the IEEE quotient
 *      for every pair (OCP e4m3fn, round to nearest even, NaN above 464);
 *   2. the fast quotient equals the IEEE quotient bit for bit wherever either
 *      has magnitude >= 2^-11 (below that both encode to a signed zero).
 *
 * Prints "pairs code_mismatches big_quotient_mismatches small_quotient_mismatches"
 * and exits 0 when claims 1 and 2 hold.
 * Build: gcc -O2 -fopenmp -ffp-contract=off quotient_check.c -lm
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float f_of(uint32_t b) {
  float f;
  memcpy(&f, &b, 4);
  return f;
}
static uint32_t b_of(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return b;
}

/* OCP FP8 v1.0 E4M3 encode: RNE on the exponent|mantissa field, subnormals
 * m * 2^-9, NaN (0x7F) above 464, sign carried. */
static uint32_t e4m3(float f) {
  const uint32_t b = b_of(f), sign = (b >> 24) & 0x80u, mb = b & 0x7FFFFFFFu;
  const float mag = f_of(mb);
  uint32_t c;
  if (!(mag <= 464.0f))
    c = 0x7Fu;
  else if (mag < 0.015625f)
    c = (uint32_t)rintf(mag * 512.0f);
  else
    c = ((mb + 0x7FFFFu + ((mb >> 20) & 1u)) >> 20) - 960u;
  return c | sign;
}

int main(void) {
  const float recip = 1.0f / 448.0f;
  const float clampmin = 1e-12f;
  const float tiny = 0x1p-11f;
  unsigned long long pairs = 0, bad_code = 0, bad_big = 0, bad_small = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : pairs, bad_code, bad_big, bad_small)
  for (uint32_t a = 0; a < 0x7F80u; ++a) {
    volatile float s0 = fmaxf(f_of(a << 16), clampmin);
    const float scale = s0 * recip;
    volatile float one = 1.0f;
    const float r = one / scale;
    for (uint32_t xb = 0; xb < 65536u; ++xb) {
      if ((xb & 0x7FFFu) > a) continue;
      const float x = f_of(xb << 16);
      const float exact = x / scale;
      const float q0 = x * r;
      const float e = fmaf(-q0, scale, x);
      const float q = copysignf(fmaf(e, r, q0), x);
      ++pairs;
      if (e4m3(q) != e4m3(exact)) ++bad_code;
      if (b_of(q) != b_of(exact)) {
        if (fabsf(q) >= tiny || fabsf(exact) >= tiny)
          ++bad_big;
        else
          ++bad_small;
      }
    }
  }
  printf("%llu %llu %llu %llu\n", pairs, bad_code, bad_big, bad_small);
  return (bad_code || bad_big) ? 1 : 0;
}
