/* Host check of the quantizer's division-free quotient (lt_numerics.h: lt_q8_quotient)
 * against IEEE division, over every positive finite fp16 scale dq and, for each, x at
 * and around every half-integer multiple (k + 1/2) * dq for |k| <= 140 (where rint's
 * decision flips) plus pseudo-random x over the quantizer's range and over wide exponent
 * ranges.  Prints: cases, bit mismatches among normal quotients, quantized-value
 * mismatches among all cases. */
#include <stdio.h>
#include <stdint.h>
#include <math.h>
#include "../../llamatov_amd/csrc/lt_numerics.h"

static uint64_t rng = 0x9E3779B97F4A7C15ull;
static uint32_t next32(void) {
  rng ^= rng << 13; rng ^= rng >> 7; rng ^= rng << 17;
  return (uint32_t)(rng >> 11);
}

static long long cases = 0, bad_bits = 0, bad_q = 0;

static void check(float x, float dq, float r) {
  if (!isfinite(x)) return;
  cases++;
  const float want = x / dq;
  const float got = lt_q8_quotient(x, dq, r);
  if (fabsf(want) >= 0x1p-126f && isfinite(want) && lt_f2u(want) != lt_f2u(got)) {
    if (bad_bits < 5) fprintf(stderr, "bits: x=%a dq=%a want=%a got=%a\n", x, dq, want, got);
    bad_bits++;
  }
  if (lt_q8_round_clamp(want) != lt_q8_round_clamp(got)) {
    if (bad_q < 5) fprintf(stderr, "q: x=%a dq=%a want=%a got=%a\n", x, dq, want, got);
    bad_q++;
  }
}

int main(void) {
  for (uint32_t h = 1; h < 0x7C00u; h++) {
    const float dq = lt_half_to_float_bits((uint16_t)h);
    const float r = 1.0f / dq;
    for (int k = -140; k <= 140; k++) {
      const float base = ((float)k + 0.5f) * dq;   /* exact: 9-bit by 11-bit significands */
      const uint32_t b = lt_f2u(base);
      for (int d = -3; d <= 3; d++) check(lt_u2f(b + (uint32_t)d), dq, r);
      check((float)k * dq, dq, r);
    }
    for (int i = 0; i < 256; i++) {
      const float u = (float)(int32_t)next32() * 0x1p-31f;        /* [-1, 1) */
      check(u * 130.0f * dq, dq, r);
      const int e = (int)(next32() % 200u) - 100;                  /* wide exponents */
      check(ldexpf(1.0f + 0.5f * u, e) * dq, dq, r);
    }
  }
  printf("%lld %lld %lld\n", cases, bad_bits, bad_q);
  return 0;
}
