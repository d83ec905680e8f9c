// llz_xform.h -- the logits as the sampler sees them.
//
// The reference's decode loop post-processes the final logits before
// Sampler.sample (main.zig:653-666): soft-capping v = tanh(v / s) * s when
// s > 0, then the logit scale v *= 1 / scale when scale is neither 1 nor 0.
// sampleWithRandom then applies the repetition penalty to a copy
// (sampler.zig:54-75).  RowSrc applies all three to a caller's row at every
// read, so the kernels read each logit from HBM as the caller wrote it and
// see the values the reference computes with:
//   at(i) / load4  -- penalised post-processed logits (the chain's input);
//   pre(v)         -- post-processing only (sampleArgmax's input at
//                     sampler.zig:50,89 is `logits`, not `penalized`).
// The penalised positions of a row (the distinct ids < n among the last
// min(len, window) history tokens, at most kPenMax of them) are collected
// once per row into LDS (pen_build), sorted; a read checks membership there.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "llz_internal.h"
#include "llz_math.h"
#include "llz_norm.h"
#include "llz_wg.h"

namespace llz {

// A row's logits through a global-address-space pointer.  The readers below
// also run inside out-of-line functions, where a generic pointer makes flat
// loads, which count on the LDS counter too: every LDS wait there would then
// also wait for the row's loads in flight.
__device__ __forceinline__ const __attribute__((address_space(1))) float* grow(const float* x) {
  return (const __attribute__((address_space(1))) float*)x;
}

// main.zig:653-666 on one logit.
__device__ __forceinline__ float logit_post(float v, uint32_t xf, float cap, float inv_scale) {
  if (xf & kXfCap) v = tanh_f32(v / cap) * cap;
  if (xf & kXfScale) v = v * inv_scale;
  return v;
}

// sampler.zig:65-69 on a logit of a penalised position.
__device__ __forceinline__ float penalise(float v, float rp) { return v > 0.0f ? v / rp : v * rp; }

// Soft-capped rows (kXmCap): the single pass's estimate of a logit's
// post-processed value f(r) = RN(RN(tanh(RN(r / cap)) cap) inv) from the
// closed form C tanh(z) = C - 2C / (exp(2z) + 1), z = r / cap, C = cap inv:
//   v~ = RN(RN(rc (-2C)) + C),  rc = rcp(RN(exp2(RN(r a2)) + 1)),
//   a2 = RN(2 log2(e) / cap),
// one hardware exp2 and one reciprocal where the exact tanh takes some sixty
// operations.  Error against f (first order, in units of C 2^-24, the
// hardware exp2 and rcp within 1 ulp):
//   v~ against C tanh(z): the exp2 argument's two roundings and the exp2
//   move 1 / (e^(2z) + 1) by a relative (|2z| + 1) 2^-23 (1 - rho), rho =
//   1 / (e^(2z) + 1), and 2 rho (1 - rho) (|2z| + 1) 2^-23 <= 1.6 units;
//   the sum's rounding and the reciprocal add 2 rho 3 2^-24 <= 6; C's
//   rounding, the product's (|2C rc| 2^-24 <= 2 units) and the sum's 4:
//   11.6 units;
//   f against C tanh(z): RN(r / cap) moves tanh by at most max z sech^2 z
//   < 0.45 units; tanh_f32 is within 3 units of tanh (checked on every
//   float); the two products' roundings add 1 unit each: 6.45 units;
// so |v~ - f| < 20 C 2^-24.  A penalised position's estimate pen_est(v~)
// (sampler.zig:65-69 with a multiply by RN(1 / rp)) lies within
// max(1, rp, 1 / rp) (2 * 20 + 3) C 2^-24 of the reference's value (the
// doubled term covers a sign that v~ and f do not share; the 3 units are
// RN(1 / rp) and the two sides' roundings).  The host turns the bound
// (taken as 44 units with the penalty) into est_xe = l2e_t * bound, the
// estimates' extra relative error (exp2 of an argument off by l2e_t |dv| is
// off by ln 2 l2e_t |dv| to first order; the factor 1 / ln 2 covers the
// rest), and takes the single pass only where est_xe <= 2^-11.
__device__ __forceinline__ float cap_est(float r, float a2, float c) {
  const float e = __builtin_amdgcn_exp2f(r * a2);
  const float rc = __builtin_amdgcn_rcpf(e + 1.0f);
  return rc * (-2.0f * c) + c;  // a product and a sum: one uniform operand each (an fma would hold -2C in a VGPR)
}
__device__ __forceinline__ float pen_est(float v, float rp, float rp_inv) { return v > 0.0f ? v * rp_inv : v * rp; }

// The penalised positions of one row, ascending, and for each of the
// single-pass kernel's eight waves the segments (256 logits; wave w owns
// segments w, w + 8, ...) holding one: bit k of wmask[w] for segment w + 8k.
struct PenShared {
  uint32_t pos[kPenMax];
  uint64_t wmask[8];
  int n;
};

// The row's penalty window as lane j's id j (0xffffffff past the window):
// one load, issued early by the caller so that it lands while other work
// goes on.
__device__ __forceinline__ uint32_t pen_window_id(const RowParams& P, const RowPtrs& Q, int row) {
  const int lane = lane_id();
  const uint32_t* win = Q.prev_win + (int64_t)row * P.prev_stride;
  return lane < P.pen_w ? win[lane] : 0xffffffffu;
}

// Wave 0 writes the row's penalised positions to LDS, ascending, with the
// waves' segment masks: lane j holds the window's id j, with bit 31 set
// unless it is the first occurrence of an id < n (sampler.zig:62-70
// penalises each id once; ids >= n never match, :64).  The caller
// synchronises the workgroup before any read uses them.
__device__ __forceinline__ void pen_list(PenShared& ps, uint32_t idf) {
  if (wave_id() != 0) return;
  const int lane = lane_id();
  const bool first = (idf >> 31) == 0u;
  const uint32_t id = idf & 0x7fffffffu;
  const uint64_t km = bal64(first);
  uint32_t rank = 0;
  uint64_t wm = 0;
  for (uint64_t bm = km; bm != 0ull; bm &= bm - 1ull) {
    const uint32_t o = readlane_u32(id, __ffsll((long long)bm) - 1);
    rank += o < id ? 1u : 0u;
    const uint32_t g = o >> 8;  // its segment
    if ((int)(g & 7u) == lane && (g >> 3) < 64u) wm |= 1ull << (g >> 3);
  }
  if (first) ps.pos[rank] = id;
  if (lane == 0) ps.n = __popcll(km);
  if (lane < 8) ps.wmask[lane] = wm;
}

// A row of logits as the chain reads it (see the file comment).  CAP =
// false: a row whose transforms include no soft-capping (kXmLight), without
// the tanh code, which a kernel would otherwise carry (and hold registers
// for) wherever it reads the row.
template <bool CAP>
struct RowSrcT {
  const float* x;       // the row as the caller passed it
  uint32_t xf;          // kXf* bits applied on reads through at() / load4()
  float cap, inv_scale, rp;
  const PenShared* pen; // penalised positions (kXfPen)

  __device__ __forceinline__ float pre(float v) const {
    if constexpr (CAP) {
      return logit_post(v, xf, cap, inv_scale);
    } else {
      return (xf & kXfScale) ? v * inv_scale : v;
    }
  }

  __device__ __forceinline__ bool penalised(int i) const {
    // the segment's bit first (one LDS read; most segments hold none)
    const uint32_t g = (uint32_t)i >> 8;
    if ((g >> 3) < 64u && ((pen->wmask[g & 7u] >> (g >> 3)) & 1ull) == 0ull) return false;
    const int np = pen->n;
    // lower bound of i in the sorted list
    int lo = 0, hi = np;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (pen->pos[mid] < (uint32_t)i) lo = mid + 1; else hi = mid;
    }
    return lo < np && pen->pos[lo] == (uint32_t)i;
  }

  // One read value v of position i through the row's transforms.
  __device__ __forceinline__ float fix(int i, float v) const {
    if (xf == 0u) return v;
    v = pre(v);
    if ((xf & kXfPen) && penalised(i)) v = penalise(v, rp);
    return v;
  }

  __device__ __forceinline__ float at(int i) const { return fix(i, grow(x)[i]); }

  // Four consecutive read values from position pos; positions >= n are left
  // as they are (callers fill them with their own neutral value).  pre4:
  // post-processing only; pen4: the penalty only; fix4: both.
  __device__ __forceinline__ float4 pre4(int pos, float4 v, int n) const {
    if ((xf & (kXfCap | kXfScale)) == 0u) return v;
    v.x = pos + 0 < n ? pre(v.x) : v.x;
    v.y = pos + 1 < n ? pre(v.y) : v.y;
    v.z = pos + 2 < n ? pre(v.z) : v.z;
    v.w = pos + 3 < n ? pre(v.w) : v.w;
    return v;
  }
  __device__ __forceinline__ float4 pen4(int pos, float4 v, int n) const {
    if ((xf & kXfPen) == 0u) return v;
    v.x = pos + 0 < n && penalised(pos + 0) ? penalise(v.x, rp) : v.x;
    v.y = pos + 1 < n && penalised(pos + 1) ? penalise(v.y, rp) : v.y;
    v.z = pos + 2 < n && penalised(pos + 2) ? penalise(v.z, rp) : v.z;
    v.w = pos + 3 < n && penalised(pos + 3) ? penalise(v.w, rp) : v.w;
    return v;
  }
  __device__ __forceinline__ float4 fix4(int pos, float4 v, int n) const { return pen4(pos, pre4(pos, v, n), n); }

  // kLaneV consecutive logits from pos (positions >= n read as 0).
  __device__ __forceinline__ void load4(int pos, int n, bool vec, float (&v)[kLaneV]) const {
    if (vec && pos + kLaneV <= n) {
      const llz_f4v q = *(const __attribute__((address_space(1))) llz_f4v*)(grow(x) + pos);
      v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    } else {
#pragma unroll
      for (int k = 0; k < kLaneV; ++k) v[k] = pos + k < n ? grow(x)[pos + k] : 0.0f;
    }
    if (xf != 0u) {
#pragma unroll
      for (int k = 0; k < kLaneV; ++k)
        if (pos + k < n) v[k] = fix(pos + k, v[k]);
    }
  }
};

using RowSrc = RowSrcT<true>;
using LightSrc = RowSrcT<false>;

// A row read as it is (no post-processing, no fused penalty): the same
// interface as RowSrc with no transform code, so kernels that do not
// transform compile as if they read the pointer directly.
struct PlainSrc {
  const float* x;
  __device__ __forceinline__ float pre(float v) const { return v; }
  __device__ __forceinline__ float fix(int, float v) const { return v; }
  __device__ __forceinline__ float at(int i) const { return grow(x)[i]; }
  __device__ __forceinline__ float4 pre4(int, float4 v, int) const { return v; }
  __device__ __forceinline__ float4 pen4(int, float4 v, int) const { return v; }
  __device__ __forceinline__ float4 fix4(int, float4 v, int) const { return v; }
  __device__ __forceinline__ void load4(int pos, int n, bool vec, float (&v)[kLaneV]) const {
    if (vec && pos + kLaneV <= n) {
      const llz_f4v q = *(const __attribute__((address_space(1))) llz_f4v*)(grow(x) + pos);
      v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    } else {
#pragma unroll
      for (int k = 0; k < kLaneV; ++k) v[k] = pos + k < n ? grow(x)[pos + k] : 0.0f;
    }
  }
};

// The chain's view of row `row` (src: the caller's rows, or the penalised
// copy) and sampleArgmax's view (the caller's rows, post-processing only).
template <bool CAP = true>
__device__ __forceinline__ RowSrcT<CAP> row_src(const RowParams& P, const RowPtrs& Q, int row, const PenShared* pen) {
  return RowSrcT<CAP>{Q.src + (int64_t)row * P.src_stride, P.xf_src, P.cap, P.inv_scale, P.rpen, pen};
}
__device__ __forceinline__ RowSrc row_orig(const RowParams& P, const RowPtrs& Q, int row) {
  return RowSrc{Q.orig + (int64_t)row * P.orig_stride, P.xf_orig & ~kXfPen, P.cap, P.inv_scale, 1.0f, nullptr};
}

}  // namespace llz
