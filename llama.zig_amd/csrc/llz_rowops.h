// llz_rowops.h -- per-row helpers shared by the kernels: workgroup maximum,
// sampleArgmax over a row, vector loads and the reference's term.
#pragma once

#include <hip/hip_runtime.h>

#include "llz_internal.h"
#include "llz_math.h"
#include "llz_norm.h"
#include "llz_wg.h"
#include "llz_xform.h"

namespace llz {

constexpr int kNT = 512;           // threads of the per-row workgroup
constexpr int kV = kLaneV;         // logits per thread per streaming tile
constexpr int kTile = kNT * kV;    // 4096 logits per tile
constexpr int kCap = kCandCap;     // candidate list capacity (power of two)
constexpr float kInf = __builtin_inff();

// ---------------------------------------------------------------------------
// small helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_fmax(float v) {
  const uint32_t r = wave_incl_scan_op(__float_as_uint(v), __float_as_uint(-kInf), [](uint32_t a, uint32_t b) {
    return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
  });
  return __uint_as_float(lane_readlast(r));
}

template <int NT>
__device__ __forceinline__ float wg_fmax(float v, WgScratch<NT>& sh, int& bank) {
  v = wave_fmax(v);
  if (lane_id() == 0) sh.red[bank][wave_id()] = __float_as_uint(v);
  lds_barrier();
  float r = __uint_as_float(sh.red[bank][0]);
#pragma unroll
  for (int w = 1; w < WgScratch<NT>::W; ++w) r = fmaxf(r, __uint_as_float(sh.red[bank][w]));
  bank ^= 1;
  return r;
}

// (value, index) ordering of sampleArgmax (sampler.zig:31-41): larger value
// wins, equal values keep the lower index, NaN never wins.
__device__ __forceinline__ bool amax_better(float v, uint32_t i, float bv, uint32_t bi) {
  if (v != v) return false;
  if (bv != bv) return true;
  return v > bv || (v == bv && i < bi);
}

// sampleArgmax over one row with the whole workgroup.  A NaN at index 0
// is never replaced by the reference's loop, so the answer is then 0.
template <int NT, class Src>
__device__ uint32_t wg_argmax_row(const Src& x, int n, WgScratch<NT>& sh, int& bank) {
  const int t = (int)threadIdx.x;
  float bv = __builtin_nanf("");
  uint32_t bi = 0xffffffffu;
  for (int i = t; i < n; i += NT) {
    const float v = x.at(i);
    if (amax_better(v, (uint32_t)i, bv, bi)) { bv = v; bi = (uint32_t)i; }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(bv, m, kWave);
    const uint32_t oi = __shfl_xor(bi, m, kWave);
    if (amax_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  if (lane_id() == 0) {
    sh.red[bank][wave_id()] = bi;
    sh.red[bank ^ 1][wave_id()] = __float_as_uint(bv);
  }
  lds_barrier();
  float rv = __builtin_nanf("");
  uint32_t ri = 0xffffffffu;
  for (int w = 0; w < WgScratch<NT>::W; ++w) {
    const float v = __uint_as_float(sh.red[bank ^ 1][w]);
    const uint32_t i = sh.red[bank][w];
    if (amax_better(v, i, rv, ri)) { rv = v; ri = i; }
  }
  lds_barrier();  // both banks were used
  const float x0 = x.at(0);
  if (x0 != x0 || ri == 0xffffffffu) ri = 0;
  return ri;
}

// e_i = exp((v_i - max) / T) as sampler.zig:85 evaluates it.
__device__ __forceinline__ float row_exp(float v, float m, float T, bool t_is_one) {
  float x = v - m;
  if (!t_is_one) x = x / T;  // x / 1.0f == x exactly, so the divide is skipped
  return exp_f32(x);
}

}  // namespace llz
