// llz_exact.h -- exact, parallel emulation of a sequential f32 accumulation.
//
// The reference sampler accumulates in f32, one term at a time, in a fixed
// order (src/sampler.zig:83-88 normaliser, :112-117 top-p, :129-132 entropy,
// :148-153 typical cum, :156-159 total, :162-166 the draw).  Summing the same
// terms "more accurately" in parallel changes the result, so the kernels
// reproduce the sequential rounding exactly:
//
//   While the running value s stays in one binade [2^j, 2^(j+1)) its grid is
//   u = 2^(j-23), s = N*u with N an integer, and fl(s + x) = (N + RN(x/u))*u
//   unless x/u is an exact half-integer (a tie, resolved by the parity of
//   the running N) or the result leaves the binade.  Between such events the
//   accumulation is an integer sum of per-term roundings, which is
//   associative.  Each tile is therefore summed with one workgroup
//   reduction; only tiles containing an event take a slower path that
//   locates the first event with a prefix scan, performs that single f32
//   operation literally, and continues with the new grid.
//
// The subtractive chain of the draw (r -= p, stop at r <= 0) uses the same
// grid argument downwards: events are ties and results at or below the
// binade's base.
#pragma once

#include <math.h>
#include <stdint.h>

#ifdef __HIPCC__
#include <hip/hip_runtime.h>
#define LLZ_HD __host__ __device__ __forceinline__
#else
#include <string.h>
#define LLZ_HD static inline
#endif

namespace llz {

constexpr uint32_t kGridTop = 1u << 24;  // N reaching this leaves the binade (add)
constexpr uint32_t kGridBase = 1u << 23; // N at or below this leaves it (subtract)
constexpr uint32_t kSat = 1u << 25;      // saturation cap for rounded terms / sums

LLZ_HD uint32_t as_bits(float f) {
#ifdef __HIPCC__
  return __float_as_uint(f);
#else
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
#endif
}
LLZ_HD float as_float(uint32_t u) {
#ifdef __HIPCC__
  return __uint_as_float(u);
#else
  float f;
  memcpy(&f, &u, 4);
  return f;
#endif
}

// Grid of a running value s >= 0: j = max(exponent(s), -126) and
// N = s / 2^(j-23) (exact).  Zero and subnormals share the grid 2^-149.
struct Grid {
  int j;
  uint32_t N;
};

LLZ_HD Grid grid_of(float s) {
  const uint32_t b = as_bits(s) & 0x7fffffffu;
  const uint32_t E = b >> 23;
  Grid g;
  g.j = (int)(E == 0 ? 1u : E) - 127;
  g.N = E == 0 ? (b & 0x7fffffu) : ((b & 0x7fffffu) | 0x800000u);
  return g;
}

// 2^(j-23) as a float (j >= -126, so the value is >= 2^-149).
LLZ_HD float grid_ulp(int j) {
  const int e = j - 23;
  return e >= -126 ? as_float((uint32_t)(e + 127) << 23) : as_float(1u << (e + 149));
}

// N * 2^(j-23) as a float; exact for N < 2^24 (or a subnormal on the grid).
LLZ_HD float grid_value(uint32_t N, int j) { return (float)N * grid_ulp(j); }

// The bits of N * 2^(j-23) for N < 2^24 on grid j: a normal number when
// N >= 2^23, a subnormal (j = -126) below.  Integer operations only.
LLZ_HD uint32_t grid_bits(uint32_t N, int j) {
  return N >= 0x800000u ? (((uint32_t)(j + 127) << 23) + (N - 0x800000u)) : N;
}

// RN(x / 2^(j-23)) for a finite x >= 0 (sign bit ignored), saturated at
// kSat, and whether x / 2^(j-23) is an exact half-integer (a tie).  Without
// branches: a shift of 25 or more is done as 25 (which leaves 0 with no
// tie, since the significand is below 2^24), and the cases x >= 2^j
// (shift <= 0) are selected at the end.
LLZ_HD uint32_t grid_round_int(float x, int j, bool& tie) {
  const uint32_t b = as_bits(x) & 0x7fffffffu;
  const uint32_t XE = b >> 23;
  const uint32_t m = XE == 0 ? (b & 0x7fffffu) : ((b & 0x7fffffu) | 0x800000u);
  const int xe = (int)(XE == 0 ? 1u : XE) - 127;  // x = m * 2^(xe-23)
  const int d = j - xe;
  const int dd = d < 1 ? 1 : (d > 25 ? 25 : d);
  const uint32_t q = m >> dd;
  const uint32_t rem = m & ((1u << dd) - 1u);
  const uint32_t half = 1u << (dd - 1);
  const uint32_t r = q + (rem > half ? 1u : 0u);
  tie = d > 0 && rem == half;
  // d == 0: m itself; d < 0: x >= 2^(j+1) leaves the binade on its own
  return d > 0 ? r : (d == 0 ? m : (m == 0 ? 0u : kSat));
}

// grid_round_int through floating point, in about a third of the
// instructions (the result is the same for every x and j in [-126, 127]):
// y = |x| 2^(23-j) is exact (a power-of-two scaling; when it underflows, y
// < 2^-100 and the result is 0 either way).  Below 2^23, RN with ties down
// is ceil(y - 1/2): y - 1/2 is exact for y >= 1/2, and for y < 1/2 every
// value in [-1/2, 0) gives 0; y is a half-integer exactly when y - 1/2 is an
// integer.  In [2^23, 2^24) y is an integer; from 2^24 the term leaves the
// binade on its own (kSat).  tests/test_grid_round.py compares the two.
LLZ_HD uint32_t grid_round(float x, int j, bool& tie) {
  const float y = ldexpf(fabsf(x), 23 - j);
  const float t = y - 0.5f;
  const float c = ceilf(t);
  const bool fine = y < 0x1p23f;
  tie = fine && c == t;
  const float r = fine ? c : y;
  return !(y < 0x1p24f) ? kSat : (uint32_t)r;  // NaN too, as grid_round_int
}

// Largest integer T with T * 2^(j-23) <= thr, or 0xffffffff when thr is at
// or above 2^(j+1) (the running value cannot exceed it inside the binade).
// thr >= 0.
LLZ_HD uint32_t grid_floor(float thr, int j) {
  const float top = (j + 1 <= 127) ? as_float((uint32_t)(j + 1 + 127) << 23) : 3.0e38f;
  if (!(thr < top)) return 0xffffffffu;
  // thr / u < 2^24: scale by an exact power of two, then truncate
  const int e = 23 - j;  // thr * 2^e
  float scaled = thr;
  int k = e;
  while (k > 100) { scaled *= 0x1p100f; k -= 100; }
  scaled *= as_float((uint32_t)(k + 127) << 23);
  return (uint32_t)scaled;  // scaled >= 0, < 2^24: truncation == floor
}

}  // namespace llz
