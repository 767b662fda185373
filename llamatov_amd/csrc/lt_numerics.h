/* lt_numerics.h -- scalar numerics shared bit-for-bit by the gfx950 kernels and the
 * CPU restatement under oracle/.
 *
 * Everything here is written in plain C that compiles both as HIP device code
 * (hipcc, -ffp-contract=off) and as host C (gcc, -ffp-contract=off).  Every fused
 * multiply-add is written out as fma()/fmaf(); nothing relies on compiler
 * contraction, so the same source yields the same IEEE operation sequence on the
 * CPU and on the GPU, hence the same bits.
 *
 * The reference calls CUDA's expf/__expf (SiLU: bpd/lib/dev_residency.py:583,
 * attention: dev_residency.py:1994), powf/cosf/sinf (RoPE:
 * bpd/kernelgen/emitters/rope_from_facts.pl:58-60) and rsqrtf (RMSNorm:
 * bpd/kernelgen/emitters/norm_softmax_from_facts.pl:101).  Those bits are not
 * reproducible off NVIDIA hardware, so this build defines its own functions from
 * named textbook methods and bounds their error against float64 in the tests:
 *
 *   lt_expf   : Cody & Waite (1980) additive range reduction x = k*ln2 + r,
 *               |r| <= ln2/2, carried out in binary64 with a two-term ln2 split
 *               and fma; Taylor polynomial of degree 12 for e^r in binary64
 *               (truncation < 2e-16 relative); exact scaling by 2^k in binary64;
 *               one final rounding to binary32.
 *   lt_sincosf: Cody & Waite reduction by pi/2 in binary64 (two-term split,
 *               fma), quadrant selection, Taylor polynomials of degree 17 (sin)
 *               and 18 (cos) on |r| <= pi/4 in binary64, one rounding to binary32.
 *   lt_rsqrtf : binary64 sqrt and binary64 division (both correctly rounded by
 *               IEEE 754), then one rounding to binary32.
 *
 * Each result is the binary32 rounding of a binary64 value whose relative error
 * is below 1e-15, i.e. within 0.5 ulp + 1e-8 ulp of the true function value.
 */
#ifndef LT_NUMERICS_H
#define LT_NUMERICS_H

#include <stdint.h>

#if defined(__HIP__)
#define LT_HD static __host__ __device__ __forceinline__
#else
#include <math.h>
#include <string.h>
#define LT_HD static inline
#endif

/* ---- bit casts ------------------------------------------------------------------ */
LT_HD uint32_t lt_f2u(float f) { union { float f; uint32_t u; } v; v.f = f; return v.u; }
LT_HD float lt_u2f(uint32_t u) { union { float f; uint32_t u; } v; v.u = u; return v.f; }
LT_HD uint64_t lt_d2u(double d) { union { double d; uint64_t u; } v; v.d = d; return v.u; }
LT_HD double lt_u2d(uint64_t u) { union { double d; uint64_t u; } v; v.u = u; return v.d; }

/* ---- fp16 <-> fp32 (IEEE binary16, round-to-nearest-even) ------------------------- */
/* Exact widening of a binary16 bit pattern (normals, subnormals, inf, nan). */
LT_HD float lt_half_to_float_bits(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  if (exp == 0) {
    if (man == 0) return lt_u2f(sign);
    /* subnormal: value = man * 2^-24, exact in binary32 */
    float v = (float)man * lt_u2f(0x33800000u); /* 2^-24 */
    return sign ? -v : v;
  }
  if (exp == 31) return lt_u2f(sign | 0x7F800000u | (man << 13));
  return lt_u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

/* binary32 -> binary16 with round-to-nearest-even, overflow to inf, gradual underflow. */
LT_HD uint16_t lt_float_to_half_bits(float f) {
  uint32_t x = lt_f2u(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) { /* inf or nan */
    return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u | ((ax >> 13) & 0x3FFu) : 0u));
  }
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
  if (ax < 0x38800000u) {                                    /* below 2^-14: subnormal half */
    if (ax < 0x33000000u) return (uint16_t)sign;             /* < 2^-25: rounds to 0 */
    uint32_t e = ax >> 23;                                   /* biased exponent, 102..112 */
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;               /* 24-bit significand */
    uint32_t shift = 126u - e;                               /* value = m * 2^(e-150); half unit 2^-24 */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1u);
    if (rem > halfway || (rem == halfway && (q & 1u))) q += 1u;
    return (uint16_t)(sign | q);
  }
  uint32_t e = (ax >> 23) - 112u;                            /* half biased exponent 1..30 */
  uint32_t m = ax & 0x7FFFFFu;
  uint32_t q = (e << 10) | (m >> 13);
  uint32_t rem = m & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u; /* carry may bump exponent: ok */
  return (uint16_t)(sign | q);
}

/* ---- exp --------------------------------------------------------------------- */
#define LT_LN2_HI 0x1.62e42fefa39efp-1    /* binary64(ln 2) */
#define LT_LN2_LO 0x1.abc9e3b39803fp-56   /* binary64(ln 2 - LT_LN2_HI) */
#define LT_LOG2E  0x1.71547652b82fep+0    /* binary64(1 / ln 2) */

/* round half to even (the IEEE default rounding mode on both sides) */
LT_HD double lt_rint_d(double x) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_rint(x);
#else
  return rint(x);
#endif
}

LT_HD float lt_expf(float xf) {
  if (xf != xf) return xf;                 /* nan */
  if (xf > 100.0f) return lt_u2f(0x7F800000u);
  if (xf < -120.0f) return 0.0f;
  double x = (double)xf;
  double k = lt_rint_d(x * LT_LOG2E);
  double r = fma(-k, LT_LN2_HI, x);
  r = fma(-k, LT_LN2_LO, r);
  /* Taylor series of e^r, degree 12, Horner in binary64 */
  double p = 1.0 / 479001600.0;            /* 1/12! */
  p = fma(p, r, 1.0 / 39916800.0);         /* 1/11! */
  p = fma(p, r, 1.0 / 3628800.0);          /* 1/10! */
  p = fma(p, r, 1.0 / 362880.0);
  p = fma(p, r, 1.0 / 40320.0);
  p = fma(p, r, 1.0 / 5040.0);
  p = fma(p, r, 1.0 / 720.0);
  p = fma(p, r, 1.0 / 120.0);
  p = fma(p, r, 1.0 / 24.0);
  p = fma(p, r, 1.0 / 6.0);
  p = fma(p, r, 0.5);
  p = fma(p, r, 1.0);
  p = fma(p, r, 1.0);
  int ki = (int)k;                          /* |k| <= 174 here */
  double two_k = lt_u2d((uint64_t)(ki + 1023) << 52);
  return (float)(p * two_k);
}

/* lt_expf without branches: the same binary64 path on the argument clamped to [-120, 100]
 * (unchanged inside that range; a nan runs on 0), then selects give the nan, overflow and
 * underflow results of lt_expf.  Equal to lt_expf for every input; on the GPU independent
 * calls (several heads' or positions' exps) interleave instead of each running as its own
 * masked branch. */
LT_HD float lt_expf_sel(float xf) {
  const int isnan_ = xf != xf;
  const float xc = isnan_ ? 0.0f : (xf > 100.0f ? 100.0f : (xf < -120.0f ? -120.0f : xf));
  double x = (double)xc;
  double k = lt_rint_d(x * LT_LOG2E);
  double r = fma(-k, LT_LN2_HI, x);
  r = fma(-k, LT_LN2_LO, r);
  double p = 1.0 / 479001600.0;
  p = fma(p, r, 1.0 / 39916800.0);
  p = fma(p, r, 1.0 / 3628800.0);
  p = fma(p, r, 1.0 / 362880.0);
  p = fma(p, r, 1.0 / 40320.0);
  p = fma(p, r, 1.0 / 5040.0);
  p = fma(p, r, 1.0 / 720.0);
  p = fma(p, r, 1.0 / 120.0);
  p = fma(p, r, 1.0 / 24.0);
  p = fma(p, r, 1.0 / 6.0);
  p = fma(p, r, 0.5);
  p = fma(p, r, 1.0);
  p = fma(p, r, 1.0);
  int ki = (int)k;
  double two_k = lt_u2d((uint64_t)(ki + 1023) << 52);
  float v = (float)(p * two_k);
  v = xf > 100.0f ? lt_u2f(0x7F800000u) : v;
  v = xf < -120.0f ? 0.0f : v;
  return isnan_ ? xf : v;
}

/* ---- sin / cos ------------------------------------------------------------------- */
#define LT_PIO2_HI 0x1.921fb54442d18p+0   /* binary64(pi/2) */
#define LT_PIO2_LO 0x1.1a62633145c07p-54  /* binary64(pi/2 - LT_PIO2_HI) */
#define LT_2OPI    0x1.45f306dc9c883p-1   /* binary64(2/pi) */

LT_HD double lt_sin_poly(double r) {
  double r2 = r * r;
  double p = -1.0 / 355687428096000.0;     /* -1/17! */
  p = fma(p, r2, 1.0 / 1307674368000.0);   /* 1/15! */
  p = fma(p, r2, -1.0 / 6227020800.0);     /* -1/13! */
  p = fma(p, r2, 1.0 / 39916800.0);        /* 1/11! */
  p = fma(p, r2, -1.0 / 362880.0);         /* -1/9! */
  p = fma(p, r2, 1.0 / 5040.0);            /* 1/7! */
  p = fma(p, r2, -1.0 / 120.0);            /* -1/5! */
  p = fma(p, r2, 1.0 / 6.0);               /* 1/3! ... sign applied below */
  /* sin r = r - r^3/6 + ... = r - r^3 * (1/6 - r^2/120 + ...) */
  return fma(-(r * r2), p, r);
}

LT_HD double lt_cos_poly(double r) {
  double r2 = r * r;
  double p = 1.0 / 6402373705728000.0;     /* 1/18! */
  p = fma(p, r2, -1.0 / 20922789888000.0); /* -1/16! */
  p = fma(p, r2, 1.0 / 87178291200.0);     /* 1/14! */
  p = fma(p, r2, -1.0 / 479001600.0);      /* -1/12! */
  p = fma(p, r2, 1.0 / 3628800.0);         /* 1/10! */
  p = fma(p, r2, -1.0 / 40320.0);          /* -1/8! */
  p = fma(p, r2, 1.0 / 720.0);             /* 1/6! */
  p = fma(p, r2, -1.0 / 24.0);             /* -1/4! */
  p = fma(p, r2, 0.5);                     /* 1/2! ... sign applied below */
  /* cos r = 1 - r^2 * (1/2 - r^2/24 + ...) */
  return fma(-r2, p, 1.0);
}

/* sin and cos of a binary32 argument; valid (<1e-15 relative before the final
 * rounding) for |x| < 2^30, far beyond any rotary angle used here. */
LT_HD void lt_sincosf(float xf, float* s_out, float* c_out) {
  double x = (double)xf;
  double k = lt_rint_d(x * LT_2OPI);
  double r = fma(-k, LT_PIO2_HI, x);
  r = fma(-k, LT_PIO2_LO, r);
  double s = lt_sin_poly(r), c = lt_cos_poly(r);
  long long q = (long long)k & 3;
  double so, co;
  if (q == 0) { so = s; co = c; }
  else if (q == 1) { so = c; co = -s; }
  else if (q == 2) { so = -s; co = -c; }
  else { so = -c; co = s; }
  *s_out = (float)so;
  *c_out = (float)co;
}

/* ---- reciprocal square root ---------------------------------------------------- */
LT_HD float lt_rsqrtf(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
  return (float)(1.0 / __builtin_sqrt((double)x));
#else
  return (float)(1.0 / sqrt((double)x));
#endif
}

/* ---- activation quantization (engine convention) ----------------------------------
 * d = amax/127 (binary32 IEEE division), stored as fp16 RNE; amax == 0 -> d = 1.0;
 * q = clamp(rint(x / float(d16)), -127, 127) with ties to even.
 * Reference: bpd/lib/dev_residency.py:799-808, 867-886; fact_dispatch.py:383-391. */
LT_HD uint16_t lt_q8_scale_bits(float amax) {
  float d = (amax > 0.0f) ? amax / 127.0f : 1.0f;
  return lt_float_to_half_bits(d);
}

LT_HD float lt_rintf(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_rintf(x);
#else
  return rintf(x);
#endif
}

/* clamp(rint(v), -127, 127) with the saturating float->int conversion of the GPUs the
 * quantizer runs on: +-inf and out-of-range values saturate, NaN converts to 0. */
LT_HD int lt_q8_round_clamp(float v) {
  float t = lt_rintf(v);
  t = (t == t) ? t : 0.0f;
  return (int)fminf(fmaxf(t, -127.0f), 127.0f);
}

LT_HD int lt_q8_quant1(float x, float dq) { return lt_q8_round_clamp(x / dq); }

/* x / dq without a division per element, for r = RN(1/dq) (one IEEE division per block).
 * q = RN(x*r) is within 2 ulp of x/dq; each step q' = RN(q + RN(x - q*dq) * r) uses the
 * residual x - q*dq, which fma computes exactly when q is within 2 ulp.  Markstein (1990,
 * "Computation of elementary functions on the IBM RISC System/6000 processor"): when r is
 * the correctly rounded reciprocal and q is faithful, one step yields the correctly rounded
 * quotient; the first step makes q faithful, the second rounds it correctly.  For finite
 * nonzero dq and finite x this equals x / dq bit for bit whenever |x / dq| is a normal
 * number (below that, both round to an integer 0 in the quantizer); dq = inf gives NaN
 * here and +-0 in IEEE division, both of which the quantizer maps to 0. */
LT_HD float lt_q8_quotient(float x, float dq, float r) {
  float q = x * r;
  q = fmaf(fmaf(-q, dq, x), r, q);
  return fmaf(fmaf(-q, dq, x), r, q);
}

/* SiLU(g) * u exactly as the reference writes it: (g / (1 + exp(-g))) * u.
 * Reference: bpd/lib/dev_residency.py:583. */
LT_HD float lt_silu_mul(float g, float u) {
  return (g / (1.0f + lt_expf(-g))) * u;
}

#endif /* LT_NUMERICS_H */
