// llz_norm.h -- the row normaliser (sampler.zig:83-88) at streaming speed.
//
//   sum = 0;  for i in 0..n:  e_i = exp((v_i - max) / T);  sum += e_i   (f32)
//
// With the running sum s in binade j (grid u = 2^(j-23)), term i adds the
// integer r_i = RN(e_i / u) unless that quotient is an exact half-integer
// (a tie) or the sum leaves the binade (llz_exact.h).  The kernel computes
// r_i without the exact exp for almost every element:
//
//   q_i = exp2(RN(v_i - max) * log2(e)/T + 23 - j)      (hardware exp2)
//
// approximates e_i / u with relative error below kEps (bound below).  When
// q_i is farther than q_i * kEps from every half-integer, RN(e_i / u) equals
// rint(q_i) exactly.  The remaining "special" elements -- ambiguous
// roundings, large terms (q >= ~2^15) and candidates for the sorted list --
// go through a per-wave LDS queue and are evaluated with the exact exp
// (llz_math.h) by dense lanes.
//
// Error bound (relevant elements have q in [2^-2, 2^15] and the grid is kept
// to j >= -40): t = RN(d * RN(log2(e)/T) + 23 - j) with d = RN(v - max)
// exactly as the reference computes it.  |t - (x log2 e + 23 - j)| <= 2^-20
// (rounding of t, |t| < 16) + 2^-18 (RN of log2(e)/T times |d log2 e/T| <=
// 65) + 2^-18.5 (x = RN(d/T) vs d/T, |x| < 45) < 2^-17, i.e. 5.3e-6 relative
// in q; the hardware exp2 adds < 8.5e-8 (measured over every f32 input in
// [-40, 40]) and the reference exp < 1.2e-7.  kEps = 2^-16 = 1.5e-5.
//
// Events (ties, binade crossings) are located per 256-element wave chunk:
// per-chunk integer sums of a group of tiles are scanned by one wave, and
// only the wave owning the first event chunk replays it exactly.
#pragma once

#include "llz_accum.h"
#include "llz_math.h"
#include "llz_wg.h"

namespace llz {

constexpr float kEps = 0x1p-16f;
constexpr int kPrologue = 64;   // elements summed by wave 0 before the tiled loop

__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
__device__ __forceinline__ float readlane_f32(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Wave-level exact accumulation (add) of V terms per lane, lane-major order
// (lane l holds positions l*V .. l*V+V-1).  Absent terms have the sign bit
// set.  All lanes return the same value.
template <int V>
__device__ float wave_accumulate(float s, const float (&x)[V]) {
  const int lane = lane_id();
  int done = -1;
  for (;;) {
    const Grid g = grid_of(s);
    uint32_t r[V];
    bool tie[V];
    uint32_t tsum = 0;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int p = lane * V + k;
      r[k] = 0;
      tie[k] = false;
      if (p > done && !(as_bits(x[k]) >> 31)) r[k] = grid_round(x[k], g.j, tie[k]);
      tsum = sat_add(tsum, r[k], kSat);
    }
    const uint32_t incl = wave_incl_scan_sat(tsum, kSat);
    const uint32_t excl = wave_shift_up1(incl);
    uint32_t run = g.N + excl;
    int my_evt = -1;
    uint32_t my_before = 0;
    float my_x = 0.0f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int p = lane * V + k;
      if (my_evt < 0 && p > done && !(as_bits(x[k]) >> 31)) {
        const uint32_t before = run;
        run += r[k];
        if (tie[k] || run >= kGridTop) {
          my_evt = p;
          my_before = before;
          my_x = x[k];
        }
      }
    }
    const uint64_t mask = bal64(my_evt >= 0);
    if (mask == 0ull) return grid_value(g.N + readlane_u32(incl, kWave - 1), g.j);
    const int L = __ffsll((long long)mask) - 1;
    const int P = (int)readlane_u32((uint32_t)my_evt, L);
    s = grid_value(readlane_u32(my_before, L), g.j) + readlane_f32(my_x, L);
    done = P;
    if (done >= kWave * V - 1) return s;
  }
}

// The chain of one 64-term chunk, the terms held one per lane (lane i: term
// i, i < len <= 64; absent terms have the sign bit set): lane i < len ends
// with the running value after term i (lanes from len on hold no useful
// value).  Lane 0 starts as s + x_0 and every other lane as its own term;
// each step adds to every lane the value of the lane below it (one DPP
// instruction, wave_shr:1), so lane i holds the sequential chain through
// term i from step i on and keeps it: (value after term i-1) + x_i is the
// reference's own next operation.  SUB subtracts: s - x is computed as s +
// (-x), which IEEE defines to be the same.
template <bool SUB>
__device__ __forceinline__ float wave_chain_lanes(float s, float x0, int len) {
  const int lane = lane_id();
  const bool present = lane < len && !(as_bits(x0) >> 31);
  const float x = present ? (SUB ? -x0 : x0) : -0.0f;
  const float y = lane == 0 ? s + x : x;
  float acc = y;
  // steps in groups of eight (a step past len leaves lanes < len unchanged)
#pragma unroll
  for (int k8 = 1; k8 < kWave; k8 += 8) {
    if (k8 >= len) break;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      acc = y + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0x138, 0xf, 0xf, true));
  }
  return acc;
}

// Sequential accumulation over a short list by one wave (the reference's
// loop, one term at a time).  ADD stops at the first s > thr (thr >= 0),
// SUB at the first s <= 0; absent terms (sign bit set) are skipped.  Chunk by
// chunk of 64 (wave_chain_lanes), one ballot per chunk for the first stop.
template <bool SUB, typename TermFn>
__device__ float wave_seq_list(float s, int len, float thr, int& stop, TermFn term) {
  stop = -1;
  const int lane = lane_id();
  for (int base = 0; base < len; base += kWave) {
    const int p = base + lane;
    const float x0 = p < len ? term(p) : -0.0f;
    const int cnt = min(kWave, len - base);
    const bool present = lane < cnt && !(as_bits(x0) >> 31);
    const float acc = wave_chain_lanes<SUB>(s, x0, cnt);
    const bool hit = present && (SUB ? (acc <= 0.0f) : (thr >= 0.0f && acc > thr));
    const uint64_t hits = bal64(hit);
    if (hits != 0ull) {
      const int L = __ffsll((long long)hits) - 1;
      stop = base + L;
      return readlane_f32(acc, L);
    }
    s = readlane_f32(acc, cnt - 1);
  }
  return s;
}

constexpr int kLaneV = 4;                  // logits per lane per sub-chunk (one float4)
constexpr int kSub = 4;                    // float4 sub-chunks per lane per group
constexpr int kSlice = kWave * 4 * kSub;   // 1024 elements: one wave's slice of a group
constexpr int kQCap = 512;                 // special queue capacity per wave

// Shared memory of the normaliser (reused by later stages).
template <int NT>
struct NormShared {
  static constexpr int W = NT / kWave;
  float ev[W][kSub * kLaneV][kWave];   // per element slot: logit in, exact term out (specials only)
  uint16_t q[W][kQCap];            // queue of special element slots (c*kV + k) * 64 + lane
  uint32_t part[2][W * kSub + 1];  // sub-chunk sums of a group (bit 31: event), groups alternate;
                                   // the extra word carries a resolution's status
  float s_bcast[2];                // running sum broadcast
};

// N + incl >= 2^24: the running sum leaves the binade within this prefix.
__device__ __forceinline__ bool g_top_reached(uint32_t N, uint32_t incl) { return N + incl >= kGridTop; }

// x = RN(v - max) / T exactly as sampler.zig:85 evaluates it
__device__ __forceinline__ float exact_term(float v, float m, float T, bool t1) {
  float x = v - m;
  if (!t1) x = x / T;
  return exp_f32(x);
}

// Approximate q = e / 2^(j-23): rq = rint(min(q, 2^15)) is RN(e / u) unless
// the element is special (ambiguous rounding, q >= 2^15 or a candidate,
// q >= qc).  Deterministic, so a second evaluation gives the same rq.
struct Approx {
  float rq;
  bool special;
};

__device__ __forceinline__ Approx approx_term(float v, float m, float L2E_T, float cj, float qc) {
  const float d = v - m;
  const float t = fmaf(d, L2E_T, cj);
  const float q = __builtin_amdgcn_exp2f(t);
  const float rq = rintf(fminf(q, 32768.0f));
  const float z = fabsf(q - rq);
  const bool amb = !(fmaf(q, kEps, z) < 0.5f);  // NaN-safe: unknown -> exact
  Approx a;
  a.special = amb || q >= qc;
  a.rq = rq;
  return a;
}

}  // namespace llz
