/* CPU check of the quotient used by the MuonLP kernels (lp.hip, lp_codes8): for
 * r = 1 / b (IEEE, correctly rounded), q0 = a * r, e = fma(-b, q0, a), y = fma(e, r, q0)
 * equals the IEEE quotient a / b whenever |a| <= b, b <= 2^125 and
 * |a| >= max(2^-78, b * 2^-100) (the kernels' fast-path condition). Quotients above 1 (the
 * fp8 scale is absmax / 448, so |a| / b <= 448) reduce to that case: a = 2^k a' with a' in
 * (b / 2, b] scales q0, e and y by exactly 2^k while they stay normal. The random pairs
 * test them directly too, with |a| up to 448 b.
 * Usage: markstein_check <random pairs> <exhaustive scales (0..8)>; exit status 1 on a
 * mismatch. */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static int check(float a, float b, float r, float lim, long* n) {
  if (!(fabsf(a) >= lim)) return 0;
  const float q0 = a * r, e = fmaf(-b, q0, a), y = fmaf(e, r, q0), ref = a / b;
  ++*n;
  if (f2u(y) != f2u(ref)) {
    printf("mismatch: a=%a b=%a y=%a a/b=%a\n", a, b, y, ref);
    return 1;
  }
  return 0;
}

int main(int argc, char** argv) {
  const long pairs = argc > 1 ? atol(argv[1]) : 1000000;
  const int nscales = argc > 2 ? atoi(argv[2]) : 2;
  long n = 0, bad = 0;
  /* every |a| in [lim, b] for scales with all-zero and all-ones mantissas and odd values */
  const float bs[8] = {0x1.fffffep-1f, 1.0f, 1e-12f, 3.0f, 0x1.5555p+7f, 0x1.fffffep+40f,
                       0x1.000002p-20f, 0x1.8p+100f};
  for (int i = 0; i < nscales && i < 8; ++i) {
    const float b = bs[i], r = 1.0f / b, lim = fmaxf(0x1p-78f, b * 0x1p-100f);
    for (uint32_t u = f2u(lim); u <= f2u(b); ++u) {
      bad += check(u2f(u), b, r, lim, &n);
      bad += check(-u2f(u), b, r, lim, &n);
      if (bad > 10) return 1;
    }
  }
  /* random scales in [1e-12, 2^125], random |a| over 40 binades below b and, for one pair in
   * four, up to 448 b (the fp8 range) */
  uint64_t s = 0x9e3779b97f4a7c15ull;
  for (long k = 0; k < pairs; ++k) {
    s ^= s << 13; s ^= s >> 7; s ^= s << 17;
    float b = ldexpf(1.0f + (float)(s & 0x7fffff) / 8388608.0f, (int)((s >> 23) % 166) - 40);
    if (b < 1e-12f) b = 1e-12f;
    if (b > 0x1p125f) b = 0x1p125f;
    s ^= s << 13; s ^= s >> 7; s ^= s << 17;
    const int up = ((s >> 61) & 3) == 0 ? 9 : 0;
    const double top = up ? fmin(448.0 * (double)b, (double)FLT_MAX) : (double)b;
    double ad = ldexp(1.0 + (double)(s & 0x7fffff) / 8388608.0, ilogbf(b) + up - (int)((s >> 23) % 40));
    float a = (float)fmin(ad, top);
    if (s >> 63) a = -a;
    const float r = 1.0f / b, lim = fmaxf(0x1p-78f, b * 0x1p-100f);
    bad += check(a, b, r, lim, &n);
    if (bad > 10) return 1;
  }
  printf("checked %ld quotients, %ld mismatches\n", n, bad);
  return bad != 0;
}
