/* CPU check of the quantiser quotient the kernels use (gdnr_device.h,
 * quotient_rn): q = RN(x * RN(1/s)), then two corrections with the negated
 * residual, q = fma(-fma(q, s, -x), r, q), must equal the IEEE
 * quotient x / s bit for bit on the blocks that take it (amax finite,
 * s = amax / 448 >= 2^-64, |x| <= amax). glibc's fmaf is exact, like the
 * GPU's fused multiply-add. Exit status 1 on any mismatch.
 * Usage: quotient_rn_check <random samples> <adversarial samples per divisor> */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static uint64_t st = 0x9E3779B97F4A7C15ull;
static uint64_t rnd(void) { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return st; }

static float quotient_rn(float x, float s, float r) {
  float q = x * r;
  q = fmaf(-fmaf(q, s, -x), r, q);
  q = fmaf(-fmaf(q, s, -x), r, q);
  return q;
}

static long mismatches = 0, checked = 0;
static void check(float x, float s) {
  const float r = 1.0f / s;
  const float a = quotient_rn(x, s, r), b = x / s;
  ++checked;
  if (f2u(a) != f2u(b)) {
    if (mismatches < 10) fprintf(stderr, "x=%a s=%a: %a != %a\n", x, s, a, b);
    ++mismatches;
  }
}

int main(int argc, char** argv) {
  const long n_random = argc > 1 ? atol(argv[1]) : 1000000;
  const long n_adv = argc > 2 ? atol(argv[2]) : 1000;
  /* blocks as the quantiser forms them: s = amax/448 over the whole normal
   * range s >= 2^-64, x uniform in [-amax, amax], plus x = +-amax, +-0 */
  for (long i = 0; i < n_random; ++i) {
    const float amax = u2f(((uint32_t)(62 + rnd() % 190) << 23) | (uint32_t)(rnd() & 0x7FFFFF));
    const float s = amax / 448.0f;
    if (!(s >= 0x1p-64f) || isinf(amax)) continue;
    float x = amax * (float)((double)(rnd() >> 11) / 9007199254740992.0);
    if (rnd() & 1) x = -x;
    check(x, s);
    if ((i & 1023) == 0) { check(amax, s); check(-amax, s); check(0.0f, s); check(-0.0f, s); }
  }
  /* divisors with mantissas near all-ones and near powers of two, and
   * dividends whose quotients sit within a few ulp of fp32 midpoints */
  for (int k = 0; k < 2048; ++k) {
    const uint32_t mant = (k < 1024) ? (0x7FFFFFu - (uint32_t)k) : (uint32_t)(k - 1024);
    const float s = u2f((uint32_t)(120 + k % 16) << 23 | mant);
    for (long j = 0; j < n_adv; ++j) {
      const uint32_t qm = (uint32_t)(rnd() & 0xFFFFFF) | 0x800000u;
      double qd = ldexp((double)qm, -23 - (int)(rnd() % 20));
      if (rnd() & 1) qd *= 1.0 + (double)((int)(rnd() % 9) - 4) * 0x1p-24;
      const float x = (float)(qd * (double)s);
      if (fabsf(x) <= 448.0f * s) check(rnd() & 1 ? -x : x, s);
    }
  }
  printf("%ld quotients checked, %ld mismatches\n", checked, mismatches);
  return mismatches ? 1 : 0;
}
