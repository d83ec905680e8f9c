// llz_math.h -- bit-exact f32 exp/log for the sampling kernels.
//
// The reference sampler computes std.math.exp (src/sampler.zig:85) and @log
// (src/sampler.zig:131,136) in f32.  Zig lowers both to its compiler_rt
// expf/logf, which implement the FreeBSD msun e_expf.c / e_logf.c algorithms
// (Sun Microsystems 1993; musl <= 1.1.19 carries the same control flow).
// These device functions follow those published algorithms operation for
// operation.  Each f32 operation must round exactly once, so every file that
// includes this header is compiled with -ffp-contract=off, f32 denormals on,
// and IEEE (correctly rounded) division.
//
// The final logits may be soft-capped with std.math.tanh before sampling
// (main.zig:653-658); Zig's f32 tanh / expm1 are ports of musl's tanhf.c /
// expm1f.c, restated below as tanh_f32 / expm1_f32.
//
// Notices of the third-party algorithms restated here:
//   expf, logf, expm1f (FreeBSD msun e_expf.c, e_logf.c, s_expm1f.c):
//     Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
//     Developed at SunPro, a Sun Microsystems, Inc. business.
//     Permission to use, copy, modify, and distribute this software is
//     freely granted, provided that this notice is preserved.
//     (Float versions by Ian Lance Taylor, Cygnus Support.)
//   tanhf (musl src/math/tanhf.c): musl libc, Copyright (c) 2005-2020 Rich
//     Felker, et al., MIT license ("The above copyright notice and this
//     permission notice shall be included in all copies or substantial
//     portions of the Software").
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llz {

__device__ __forceinline__ uint32_t fbits(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float bitsf(uint32_t u) { return __uint_as_float(u); }

// RN(n / d) for exp_f32's rational step (n = r c and d = 2 - c with |r| <=
// 0.35 ln2-reduced, so d in [1.6, 2.4]) by Markstein's method (P. Markstein,
// "Computation of elementary functions on the IBM RISC System/6000
// processor", IBM J. Res. Develop. 34(1), 1990): one Newton step on the
// hardware reciprocal, the quotient, its exact remainder by fma and one
// correction.  Six instructions, where the general IEEE division takes about
// twelve (scaling and fix-up for operands that cannot occur here).  exp_f32
// with it equals exp_f32 with the IEEE division on all 2^32 inputs (checked
// on the GPU); the parity tests compare it with the oracle.
__device__ __forceinline__ float div_markstein(float n, float d) {
  const float y0 = __builtin_amdgcn_rcpf(d);
  const float y1 = fmaf(fmaf(-d, y0, 1.0f), y0, y0);
  const float q0 = n * y1;
  return fmaf(fmaf(-d, q0, n), y1, q0);
}

// exp(x) for f32, e_expf.c algorithm: reduce x = k ln2 + r with a two-part
// ln2, evaluate the degree-2 rational approximation of r, scale by 2^k the
// way scalbnf does (an exact power-of-two step, then one rounding multiply).
// Written without branches: every lane evaluates the reduction with the k
// its range selects (k = 0 leaves r = x, lo = 0 exactly, as the reference's
// small-|x| branch), and the range cases are selected at the end.  Checked
// against the reference's branchy form on all 2^32 inputs.
__device__ __forceinline__ float exp_f32(float x) {
  const float ln2hi = 6.9314575195e-1f;   // 0x3f317200
  const float ln2lo = 1.4286067653e-6f;   // 0x35bfbe8e
  const float invln2 = 1.4426950216e+0f;  // 0x3fb8aa3b
  const float P1 = 1.6666625440e-1f;      // 0x3e2aaa8f
  const float P2 = -2.7667332906e-3f;     // 0xbb355215

  const uint32_t hx0 = fbits(x);
  const int sign = (int)(hx0 >> 31);
  const uint32_t hx = hx0 & 0x7fffffffu;
  // |x| > 1.5 ln2: k = (int)(x / ln2 +- 1/2); |x| in (ln2/2, 1.5 ln2]: +-1;
  // below: 0 (the clamp only matters for inputs the specials below replace)
  const float kt = fminf(fmaxf(invln2 * x + (sign ? -0.5f : 0.5f), -2.0e9f), 2.0e9f);
  const int k = hx > 0x3f851592u ? (int)kt : (hx > 0x3eb17218u ? 1 - sign - sign : 0);
  const float kf = (float)k;
  const float hi = x - kf * ln2hi;
  const float lo = kf * ln2lo;
  const float r = hi - lo;
  const float rr = r * r;
  const float c = r - rr * (P1 + rr * P2);
  const float y = 1.0f + (div_markstein(r * c, 2.0f - c) - lo + hi);
  const float s1 = k > 127 ? 0x1p127f : (k < -126 ? 0x1p-102f : 1.0f);
  const int k1 = min(max(k > 127 ? k - 127 : (k < -126 ? k + 102 : k), -126), 127);
  float res = (y * s1) * bitsf((uint32_t)(0x7f + k1) << 23);
  res = hx <= 0x39000000u ? 1.0f + x : res;                       // |x| <= 2^-13
  res = (sign && hx >= 0x42cff1b5u) ? 0.0f : res;                 // underflow to 0
  res = (!sign && hx >= 0x42b17218u) ? x * 0x1p127f : res;        // overflow
  res = hx > 0x7f800000u ? x : res;                               // NaN
  return res;
}

// log(x) for f32, e_logf.c algorithm: x = 2^k (1+f) with 1+f in
// [sqrt(2)/2, sqrt(2)), log(1+f) = f - hfsq + s (hfsq + R(z)).
__device__ __forceinline__ float log_f32(float x) {
  const float ln2_hi = 6.9313812256e-01f;  // 0x3f317180
  const float ln2_lo = 9.0580006145e-06f;  // 0x3717f7d1
  const float Lg1 = 0xaaaaaa.0p-24f;
  const float Lg2 = 0xccce13.0p-25f;
  const float Lg3 = 0x91e9ee.0p-25f;
  const float Lg4 = 0xf89e26.0p-26f;

  uint32_t ix = fbits(x);
  int k = 0;
  if (ix < 0x00800000u || (ix >> 31)) {
    if ((ix << 1) == 0) return -__builtin_inff();
    if (ix >> 31) return __builtin_nanf("");
    k -= 25;
    x *= 0x1p25f;
    ix = fbits(x);
  } else if (ix >= 0x7f800000u) {
    return x;
  } else if (ix == 0x3f800000u) {
    return 0.0f;
  }
  ix += 0x3f800000u - 0x3f3504f3u;
  k += (int)(ix >> 23) - 0x7f;
  ix = (ix & 0x007fffffu) + 0x3f3504f3u;
  x = bitsf(ix);
  const float f = x - 1.0f;
  const float s = f / (2.0f + f);
  const float z = s * s;
  const float w = z * z;
  const float t1 = w * (Lg2 + w * Lg4);
  const float t2 = z * (Lg1 + w * Lg3);
  const float R = t2 + t1;
  const float hfsq = 0.5f * f * f;
  const float dk = (float)k;
  return s * (hfsq + R) + dk * ln2_lo - hfsq + f + dk * ln2_hi;
}

}  // namespace llz

namespace llz {

// expm1(x) for f32, the s_expm1f.c algorithm as musl carries it (FreeBSD
// msun lineage, two-coefficient rational approximation): reduce x = k ln2 +
// r with a two-part ln2 and its rounding correction c, evaluate the
// approximation on r, rebuild 2^k (r - e + 1) - 1 by k's range.  Every
// operation rounds once (the file's compile flags).
__device__ __forceinline__ float expm1_f32(float x) {
  const float o_threshold = 8.8721679688e+01f;  // 0x42b17180
  const float ln2_hi = 6.9313812256e-01f;       // 0x3f317180
  const float ln2_lo = 9.0580006145e-06f;       // 0x3717f7d1
  const float invln2 = 1.4426950216e+00f;       // 0x3fb8aa3b
  const float Q1 = -3.3333212137e-2f;           // -0x888868.0p-28
  const float Q2 = 1.5807170421e-3f;            //  0xcf3010.0p-33
  const uint32_t ux = fbits(x);
  const uint32_t hx = ux & 0x7fffffffu;
  const int sign = (int)(ux >> 31);
  if (hx >= 0x4195b844u) {  // |x| >= 27 ln2, or not finite
    if (hx > 0x7f800000u) return x;
    if (sign) return -1.0f;
    if (x > o_threshold) return x * 0x1p127f;
  }
  float hi, lo, c = 0.0f;
  int k;
  if (hx > 0x3eb17218u) {    // |x| > ln2 / 2
    if (hx < 0x3f851592u) {  // and < 1.5 ln2
      if (!sign) {
        hi = x - ln2_hi;
        lo = ln2_lo;
        k = 1;
      } else {
        hi = x + ln2_hi;
        lo = -ln2_lo;
        k = -1;
      }
    } else {
      k = (int)(invln2 * x + (sign ? -0.5f : 0.5f));
      const float t = (float)k;
      hi = x - t * ln2_hi;
      lo = t * ln2_lo;
    }
    x = hi - lo;
    c = (hi - x) - lo;
  } else if (hx < 0x33000000u) {  // |x| < 2^-25
    return x;
  } else {
    k = 0;
  }
  const float hfx = 0.5f * x;
  const float hxs = x * hfx;
  const float r1 = 1.0f + hxs * (Q1 + hxs * Q2);
  const float t = 3.0f - r1 * hfx;
  float e = hxs * ((r1 - t) / (6.0f - x * t));
  if (k == 0) return x - (x * e - hxs);
  e = x * (e - c) - c;
  e -= hxs;
  if (k == -1) return 0.5f * (x - e) - 0.5f;
  if (k == 1) {
    if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
    return 1.0f + 2.0f * (x - e);
  }
  const float twopk = bitsf((uint32_t)(0x7f + k) << 23);
  if (k < 0 || k > 56) {
    float y = x - e + 1.0f;
    y = k == 128 ? y * 2.0f * 0x1p127f : y * twopk;
    return y - 1.0f;
  }
  const float tmk = bitsf((uint32_t)(0x7f - k) << 23);  // 2^-k
  return k < 23 ? (x - e + (1.0f - tmk)) * twopk : (x - (e + tmk) + 1.0f) * twopk;
}

// tanh(x) for f32, the tanhf.c algorithm as musl carries it: by |x|,
//   |x| > 10 (or NaN):         1 + 0 / |x|
//   |x| > log(3) / 2:          1 - 2 / (expm1(2|x|) + 2)
//   |x| > log(5/3) / 2:        expm1(2|x|) / (expm1(2|x|) + 2)
//   normal:                    -expm1(-2|x|) / (expm1(-2|x|) + 2)
//   subnormal or zero:         |x|
// with the sign put back.  Every lane evaluates one expm1 and one division
// with the operands its range selects (each range's operations and their
// order are the branch's own, so the value is the branchy form's bit for
// bit), which keeps the code and its live registers to one copy where a
// kernel applies it to many logits at once.
__device__ __forceinline__ float tanh_f32(float x) {
  const uint32_t ux = fbits(x);
  const uint32_t w = ux & 0x7fffffffu;
  const bool sign = (ux >> 31) != 0;
  const float ax = bitsf(w);
  const bool huge = w > 0x41200000u;  // |x| > 10, or not finite
  const bool big = w > 0x3f0c9f54u;   // |x| > log(3) / 2
  const bool mid = w > 0x3e82c578u;   // |x| > log(5/3) / 2
  const float e = expm1_f32(mid ? 2.0f * ax : -2.0f * ax);
  const float num = huge ? 0.0f : (big ? 2.0f : (mid ? e : -e));
  const float q = num / (huge ? ax : e + 2.0f);
  float t = huge ? 1.0f + q : (big ? 1.0f - q : q);
  t = w < 0x00800000u ? ax : t;  // subnormal or zero
  return sign ? -t : t;
}

}  // namespace llz
