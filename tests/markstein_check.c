/* The pack kernel's quotient: code = rint((x - min) / scale) with the division replaced
 * by Markstein's correction of a * RN(1/b):
 *     y = RN(1/b);  q0 = RN(a*y);  r = fma(-q0, b, a);  q = fma(r, y, q0)
 * This program compares q with the IEEE single-precision quotient a/b, bit for bit:
 *   - every a in [b/64, 16b] for divisors with extreme mantissas (1, 1+ulp, 2-ulp,
 *     1/15, 0.1, 1.5, ...), the codec's domain (a/b <= 15, a/b < 1/64 rounds to code 0);
 *   - `samples` random a in [b/1000, 16b] for random divisors and for scales made the way
 *     the codec makes them, span/15.
 * and, for divisors near and below FLT_MIN (spans that small are possible), the kernel's
 * whole code computation: Markstein's quotient for scale >= 2^-100, the IEEE division
 * below it; the resulting codes clamp(rint(a/b), 0, 15) must equal the division's for
 * every sampled a in [0, 16b] (subnormal a and b included), and above 2^-100 the
 * quotients themselves must be exact wherever they can round to a nonzero code.
 * Exit status 0 when nothing differs.  Usage: markstein_check [samples] [divisors]
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static uint64_t checked = 0, differ = 0;
static uint64_t rng = 88172645463325252ull;
static uint32_t next_u32(void) { rng ^= rng << 13; rng ^= rng >> 7; rng ^= rng << 17; return (uint32_t)(rng >> 16); }

static void check(float a, float b, float y) {
  volatile float ref = a / b;
  const float q0 = a * y;
  const float r = fmaf(-q0, b, a);
  const float q = fmaf(r, y, q0);
  ++checked;
  if (u_of(q) != u_of(ref) && differ++ < 5) printf("differ: a=%a b=%a q=%a a/b=%a\n", a, b, q, ref);
}

static void sweep(float b, int every, int samples) {
  volatile float one = 1.0f;
  const float y = one / b;
  if (every) {
    for (uint32_t u = u_of(b / 64.0f), hi = u_of(16.0f * b); u <= hi; ++u) check(f_of(u), b, y);
    check(0.0f, b, y);
    return;
  }
  const uint32_t lo = u_of(b / 1000.0f), hi = u_of(16.0f * b);
  for (int i = 0; i < samples; ++i) check(f_of(lo + next_u32() % (hi - lo + 1)), b, y);
}

/* the pack kernel's encode(): code of a = x - min for scale b, y = RN(1/b) */
static const float kMinFastScale = 0x1p-100f;
static float code_of(float a, float b, float y) {
  float c;
  if (b >= kMinFastScale) {
    const float q0 = a * y;
    const float r = fmaf(-q0, b, a);
    c = rintf(fmaf(r, y, q0));
  } else {
    volatile float q = a / b;
    c = rintf(q);
  }
  return fminf(fmaxf(c, 0.0f), 15.0f);
}

static uint64_t codes_checked = 0, codes_differ = 0;
static void check_code(float a, float b) {
  volatile float one = 1.0f;
  const float y = one / b;
  volatile float q = a / b;
  const float want = fminf(fmaxf(rintf(q), 0.0f), 15.0f);
  const float got = code_of(a, b, y);
  ++codes_checked;
  if (got != want && codes_differ++ < 5) printf("code differs: a=%a b=%a got %g want %g\n", a, b, got, want);
}

/* divisors from the smallest subnormal up to 2^-90, dividends anywhere in [0, 16b] */
static void small_spans(int divisors, int samples) {
  for (int i = 0; i < divisors; ++i) {
    const uint32_t e = next_u32() % 38u; /* biased exponent 0 (subnormal) .. 37 (2^-90) */
    uint32_t bu = (next_u32() & 0x7FFFFFu) | (e << 23);
    if (bu == 0) bu = 1;
    const float b = f_of(bu);
    const uint32_t hi = u_of(16.0f * b);
    for (int j = 0; j < samples; ++j) check_code(f_of(next_u32() % (hi + 1)), b);
    check_code(0.0f, b);
    check_code(15.0f * b, b);
    if (b >= kMinFastScale) { /* quotients exact where a code can be nonzero */
      volatile float one = 1.0f;
      const float y = one / b;
      const uint32_t lo = u_of(b * 0.25f);
      for (int j = 0; j < samples; ++j) check(f_of(lo + next_u32() % (hi - lo + 1)), b, y);
    }
  }
}

int main(int argc, char** argv) {
  const int samples = argc > 1 ? atoi(argv[1]) : 200000;
  const int divisors = argc > 2 ? atoi(argv[2]) : 2000;
  const float special[] = {1.0f, f_of(0x3F800001u), f_of(0x3FFFFFFFu), 1.5f, f_of(0x3FAAAAABu), 1.0f / 15.0f, 0.1f, 3.0f};
  for (unsigned i = 0; i < sizeof(special) / sizeof(special[0]); ++i) sweep(special[i], 1, 0);
  for (int i = 0; i < divisors; ++i) {
    const float b = f_of((next_u32() & 0x7FFFFFu) | ((100u + next_u32() % 60u) << 23));
    sweep(b, 0, samples);
    volatile float mx = (float)(next_u32() % 100000) / 12500.0f, mn = -(float)(next_u32() % 100000) / 12500.0f;
    volatile float span = mx - mn;
    if (span > 0.0f) sweep(span / 15.0f, 0, samples);
  }
  small_spans(divisors, samples / 4 + 1);
  printf("%llu quotients checked, %llu differ; %llu small-span codes checked, %llu differ\n",
         (unsigned long long)checked, (unsigned long long)differ, (unsigned long long)codes_checked,
         (unsigned long long)codes_differ);
  return differ != 0 || codes_differ != 0;
}
