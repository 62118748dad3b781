/* dsv4_libm.h - bit-exact restatements of the glibc 2.35 single-precision
 * functions the reference's MoE path calls (expf, log1pf), written in plain C
 * so the same source compiles for gfx950 (included by dsv4_device.h with
 * DSV4_LIBM_FN = __device__ __forceinline__) and for the host, where the CPU
 * test suite compares it with the host libm on every relevant input.
 * Compile with floating-point contraction off; the fma() calls are the only
 * fused operations.
 */
#ifndef DSV4_LIBM_H
#define DSV4_LIBM_H

#include <stdint.h>
#include <string.h>
#include <math.h>

#ifndef DSV4_LIBM_TABLE
#define DSV4_LIBM_TABLE static const
#endif

#ifndef DSV4_LIBM_FN
#define DSV4_LIBM_FN static inline
#endif

DSV4_LIBM_FN uint32_t dsv4_libm_f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
DSV4_LIBM_FN float dsv4_libm_u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
DSV4_LIBM_FN uint64_t dsv4_libm_d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
DSV4_LIBM_FN double dsv4_libm_u2d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }
DSV4_LIBM_FN float dsv4_libm_inf(void) { return dsv4_libm_u2f(0x7f800000u); }

// The reference calls glibc expf/log1pf/sqrtf (src/dsv4/dsv4_model.c:5827-5831,
// 6266). These restatements reproduce glibc's results on every input (checked
// exhaustively on the CPU against the host libm: expf over |x| < 87 and the
// over/underflow edges, log1pf over all positive finite floats).

// 2^(i/32) as double bits, minus i << 47 (the table form the exponent add
// below expects); computed from 60-digit decimal arithmetic.
DSV4_LIBM_TABLE uint64_t dsv4_libm_exp2_tab[32] = {
      0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full,
      0x3fef9301d0125b51ull, 0x3fef72b83c7d517bull, 0x3fef54873168b9aaull,
      0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, 0x3fef06fe0a31b715ull,
      0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
      0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull,
      0x3feea47eb03a5585ull, 0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull,
      0x3feea11473eb0187ull, 0x3feea589994cce13ull, 0x3feeace5422aa0dbull,
      0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
      0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull,
      0x3fef3720dcef9069ull, 0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full,
      0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

// expf: double-precision table method with 32 entries of 2^(i/32), a cubic
// polynomial, and the reduction residual r formed by one fma (the form the
// FMA-capable x86-64 libm variant computes). tab: dsv4_libm_exp2_tab or a
// copy of it (a GPU kernel keeps one in LDS).
DSV4_LIBM_FN float dsv4_libm_expf_t(float x, const uint64_t *tab) {
  if (x != x) return x + x;
  if (x > 0x1.62e42ep6f) return dsv4_libm_inf();
  if (x < -0x1.9fe368p6f) return 0.0f;
  const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
  const double shift = 0x1.8p+52;
  const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
  const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
  const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  const double xd = (double)x;
  const double z = inv_ln2_n * xd;
  double kd = z + shift;
  const uint64_t ki = dsv4_libm_d2u(kd);
  kd -= shift;
  const double r = fma(inv_ln2_n, xd, -kd);
  uint64_t t = tab[ki % 32];
  t += ki << 47;
  const double s = dsv4_libm_u2d(t);
  const double p = fma(c0, r, c1);
  const double r2 = r * r;
  double y = fma(c2, r, 1.0);
  y = fma(p, r2, y);
  y = y * s;
  return (float)y;
}

DSV4_LIBM_FN float dsv4_libm_expf(float x) { return dsv4_libm_expf_t(x, dsv4_libm_exp2_tab); }

// log1pf: argument reduction 1+x = 2^k (1+f) with a correction term, then
// log(1+f) = f - (hfsq - s(hfsq + R)), s = f/(2+f), R a degree-7 polynomial in
// s^2 (the classic single-precision log1p method). Valid for x >= 0, which is
// all the router needs (x = expf(z)).
DSV4_LIBM_FN float dsv4_libm_log1pf_nonneg(float x) {
  const float ln2_hi = dsv4_libm_u2f(0x3f317180u), ln2_lo = dsv4_libm_u2f(0x3717f7d1u);
  const float lp1 = dsv4_libm_u2f(0x3F2AAAABu), lp2 = dsv4_libm_u2f(0x3ECCCCCDu);
  const float lp3 = dsv4_libm_u2f(0x3E924925u), lp4 = dsv4_libm_u2f(0x3E638E29u);
  const float lp5 = dsv4_libm_u2f(0x3E3A3325u), lp6 = dsv4_libm_u2f(0x3E1CD04Fu);
  const float lp7 = dsv4_libm_u2f(0x3E178897u);
  const int32_t hx = (int32_t)dsv4_libm_f2u(x);
  const int32_t ax = hx & 0x7fffffff;
  if (hx >= 0x7f800000) return x + x;
  int32_t k = 1, hu = 0;
  float f = 0.0f, c = 0.0f, u;
  if (hx < 0x3ed413d7) {
    if (ax < 0x31000000) {
      if (ax < 0x24800000) return x;
      return x - x * x * 0.5f;
    }
    k = 0;
    f = x;
    hu = 1;
  }
  if (k != 0) {
    if (hx < 0x5a000000) {
      u = 1.0f + x;
      hu = (int32_t)dsv4_libm_f2u(u);
      k = (hu >> 23) - 127;
      c = (k > 0) ? 1.0f - (u - x) : x - (u - 1.0f);
      c /= u;
    } else {
      u = x;
      hu = (int32_t)dsv4_libm_f2u(u);
      k = (hu >> 23) - 127;
      c = 0.0f;
    }
    hu &= 0x007fffff;
    if (hu < 0x3504f7) {
      u = dsv4_libm_u2f((uint32_t)hu | 0x3f800000u);
    } else {
      k += 1;
      u = dsv4_libm_u2f((uint32_t)hu | 0x3f000000u);
      hu = (0x00800000 - hu) >> 2;
    }
    f = u - 1.0f;
  }
  const float hfsq = 0.5f * f * f;
  const float kf = (float)k;
  if (hu == 0) {
    if (f == 0.0f) {
      if (k == 0) return 0.0f;
      c += kf * ln2_lo;
      return kf * ln2_hi + c;
    }
    const float R = hfsq * (1.0f - 0.66666666666666666f * f);
    if (k == 0) return f - R;
    return kf * ln2_hi - ((R - (kf * ln2_lo + c)) - f);
  }
  const float s = f / (2.0f + f);
  const float z = s * s;
  const float R =
      z * (lp1 + z * (lp2 + z * (lp3 + z * (lp4 + z * (lp5 + z * (lp6 + z * lp7))))));
  if (k == 0) return f - (hfsq - s * (hfsq + R));
  return kf * ln2_hi - ((hfsq - (s * (hfsq + R) + (kf * ln2_lo + c))) - f);
}


#endif /* DSV4_LIBM_H */
