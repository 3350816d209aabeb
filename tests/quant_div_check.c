/* Exhaustive check of quant_div (cuda_inf_amd/csrc/common.h) against IEEE
 * division, the commit's quantisation x / s with s = amax / 448 + 1e-12:
 *   q0 = x r;  e = fma(-q0, s', x);  q = copysign(fma(e, r, q0), x)
 * with r = 1 / s and s' = s (s' = 0 where s is infinite).
 * 1. every finite fp16 amax and every finite fp16 x: q == x / s, bits;
 * 2. amax = inf (s = inf, r = 0, s' = 0): every finite x: q == x / s, bits;
 *    x = +-inf: a NaN of x's sign;
 * 3. x NaN, every finite amax: a NaN of x's sign, as x / s;
 * 4. controls: the method without the correction step, and without the
 *    sign, each differ from x / s somewhere (the check sees them).
 * Exit status 0 when all hold.  Built with -mfma -ffp-contract=off: every
 * product, fma and division is one IEEE operation, as on the GPU. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float h2f(uint16_t h) {
  uint32_t sg = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf((float)(m | 0x400u), (int)e - 25);
  uint32_t u;
  memcpy(&u, &v, 4);
  u |= sg;
  memcpy(&v, &u, 4);
  return v;
}
static uint32_t bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
/* variant 0: quant_div; 1: no correction step; 2: no sign fix */
static float qdiv(float x, float s, float r, int variant) {
  const float q0 = x * r;
  if (variant == 1) return q0;
  const float e = fmaf(-q0, s, x);
  const float q = fmaf(e, r, q0);
  return variant == 2 ? q : copysignf(q, x);
}
static long sweep(int variant) {
  long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(dynamic, 64)
  for (int a = 0; a < 0x7C00; a++) { /* amax +0 .. 65504 */
    const float amax = h2f((uint16_t)a);
    const float s = amax / 448.0f + 1e-12f, r = 1.0f / s;
    for (int xb = 0; xb < 0x10000; xb++) {
      if ((xb & 0x7C00) == 0x7C00) continue;
      const float x = h2f((uint16_t)xb);
      bad += bits(qdiv(x, s, r, variant)) != bits(x / s);
    }
  }
  return bad;
}
int main(void) {
  int fail = 0;
  const long bad = sweep(0);
  printf("finite amax x finite x: %ld mismatches\n", bad);
  fail |= bad != 0;
  /* 2: an infinite amax */
  {
    const float s = INFINITY / 448.0f + 1e-12f, r = 1.0f / s, s2 = 0.0f;
    long b2 = 0;
    for (int xb = 0; xb < 0x10000; xb++) {
      const float x = h2f((uint16_t)xb);
      const float q = qdiv(x, s2, r, 0);
      if ((xb & 0x7C00) != 0x7C00) b2 += bits(q) != bits(x / s);
      else if ((xb & 0x3FF) == 0) b2 += !(isnan(q) && signbit(q) == signbit(x));
    }
    printf("infinite amax: %ld mismatches\n", b2);
    fail |= b2 != 0;
  }
  /* 3: NaN x */
  {
    long b3 = 0;
    for (int a = 0; a < 0x7C00; a += 7) {
      const float amax = h2f((uint16_t)a);
      const float s = amax / 448.0f + 1e-12f, r = 1.0f / s;
      for (int xb = 0x7C01; xb < 0x10000; xb += 0x8000 - 0x400) {
        for (int m = 0; m < 0x400; m += 37) {
          const float x = h2f((uint16_t)((xb & 0x8000) | 0x7C00 | (m | 1)));
          const float q = qdiv(x, s, r, 0), d = x / s;
          b3 += !(isnan(q) && isnan(d) && signbit(q) == signbit(x) && signbit(d) == signbit(x));
        }
      }
    }
    printf("NaN x: %ld mismatches\n", b3);
    fail |= b3 != 0;
  }
  /* 4: the controls must be seen */
  const long c1 = sweep(1), c2 = sweep(2);
  printf("controls: no correction %ld, no sign %ld mismatches (both must be > 0)\n", c1, c2);
  fail |= c1 == 0 || c2 == 0;
  return fail;
}
