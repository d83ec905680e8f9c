// llz_accum.h -- workgroup-level exact sequential f32 accumulation.
//
// tile_accumulate consumes one tile of terms held V per thread (thread t
// holds tile positions t*V .. t*V+V-1, so thread order is sequence order)
// and returns the running value exactly as the sequential loop
//     for (p in 0..L) { s = s + x[p]   (or s - x[p]) ; if stop(s) break; }
// would leave it.  ADD mode may stop at the first p with s > thr (thr >= 0;
// pass a negative thr for no stop); SUB mode stops at the first s <= 0.
// A term whose sign bit is set (callers use -0.0f) is absent: it is skipped
// like an unselected token in the reference's loops (no operation, no stop
// test).  Present terms are >= +0.
// Every thread of the workgroup must call it with the same s, L and thr.
#pragma once

#include "llz_exact.h"
#include "llz_wg.h"

namespace llz {

template <int NT, int V, bool SUB>
__device__ float tile_accumulate(float s, const float (&x)[V], int L, float thr, int& stop,
                                 WgScratch<NT>& sh, int& bank) {
  const int t = (int)threadIdx.x;
  const bool has_thr = !SUB && thr >= 0.0f;
  int done = -1;
  stop = -1;
  for (;;) {
    const Grid g = grid_of(s);
    const uint32_t T = has_thr ? grid_floor(thr, g.j) : 0xffffffffu;
    const int32_t low = g.j > -126 ? (int32_t)kGridBase : 0;
    uint32_t r[V];
    bool tie[V];
    uint32_t tsum = 0;
    bool ttie = false;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int p = t * V + k;
      r[k] = 0;
      tie[k] = false;
      if (p < L && p > done && !(as_bits(x[k]) >> 31)) r[k] = grid_round(x[k], g.j, tie[k]);
      tsum = sat_add(tsum, r[k], kSat);
      ttie = ttie || tie[k];
    }
    // one barrier: per-wave saturated sums with the wave's tie flag in bit 31
    {
      const uint32_t ws = wave_sum_sat(tsum, kSat);
      const bool wt = bal64(ttie) != 0ull;
      if (lane_id() == 0) sh.red[bank][wave_id()] = ws | (wt ? 0x80000000u : 0u);
      lds_barrier();
    }
    uint32_t total = 0;
    bool anytie = false;
#pragma unroll
    for (int w = 0; w < WgScratch<NT>::W; ++w) {
      const uint32_t v = sh.red[bank][w];
      total = sat_add(total, v & 0x7fffffffu, kSat);
      anytie = anytie || (v >> 31);
    }
    bank ^= 1;

    bool fast;
    if (!SUB)
      fast = !anytie && g.N + total < kGridTop && (T == 0xffffffffu || g.N + total <= T);
    else
      fast = !anytie && (int32_t)g.N - (int32_t)total > low;
    if (fast) return grid_value(SUB ? g.N - total : g.N + total, g.j);

    // slow path: locate the first event with a prefix scan
    const uint32_t excl = wg_excl_scan_sat<NT>(tsum, kSat, sh, bank);
    int32_t run = SUB ? (int32_t)g.N - (int32_t)excl : (int32_t)(g.N + excl);
    uint32_t my_evt = 0xffffffffu;
    int32_t my_before = 0;
    float my_x = 0.0f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int p = t * V + k;
      if (p < L && p > done && !(as_bits(x[k]) >> 31) && my_evt == 0xffffffffu) {
        const int32_t before = run;
        run = SUB ? run - (int32_t)r[k] : run + (int32_t)r[k];
        bool evt = tie[k];
        if (!SUB) evt = evt || run >= (int32_t)kGridTop || (T != 0xffffffffu && (uint32_t)run > T);
        else evt = evt || run <= low;
        if (evt) {
          my_evt = (uint32_t)p;
          my_before = before;
          my_x = x[k];
        }
      }
    }
    const uint32_t P = wg_min_u32<NT>(my_evt, sh, bank);
    if (P == 0xffffffffu) {
      // unreachable when the fast test failed; keep the result well defined
      return grid_value(SUB ? g.N - total : g.N + total, g.j);
    }
    const bool owner = my_evt == P;
    float s_post = 0.0f;
    uint32_t st = 0;
    if (owner) {
      const float s_pre = grid_value((uint32_t)my_before, g.j);
      s_post = SUB ? s_pre - my_x : s_pre + my_x;
      st = SUB ? (s_post <= 0.0f) : (has_thr && s_post > thr);
    }
    wg_bcast<NT>(owner, s_post, st, sh, bank);
    if (st) {
      stop = (int)P;
      return s_post;
    }
    s = s_post;
    done = (int)P;
    if (done >= L - 1) return s;
  }
}

// Additive tile accumulation with implicit terms: R(k, j, tie) returns
// RN(term_k / 2^(j-23)) (saturated at kSat) and sets tie; E(k) returns the
// exact term, and is called only for the element at which an event is
// resolved; present(k) is false for positions outside the sequence.  Lets a
// caller supply roundings from a cheaper, exact-when-unambiguous estimate.
template <int NT, int V, typename RFn, typename EFn, typename PFn>
__device__ float tile_accumulate_fn(float s, RFn R, EFn E, PFn present, WgScratch<NT>& sh, int& bank) {
  const int t = (int)threadIdx.x;
  int done = -1;
  for (;;) {
    const Grid g = grid_of(s);
    uint32_t r[V];
    bool tie[V];
    uint32_t tsum = 0;
    bool ttie = false;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int p = t * V + k;
      r[k] = 0;
      tie[k] = false;
      if (p > done && present(k)) r[k] = R(k, g.j, tie[k]);
      tsum = sat_add(tsum, r[k], kSat);
      ttie = ttie || tie[k];
    }
    {
      const uint32_t ws = wave_sum_sat(tsum, kSat);
      const bool wt = bal64(ttie) != 0ull;
      if (lane_id() == 0) sh.red[bank][wave_id()] = ws | (wt ? 0x80000000u : 0u);
      lds_barrier();
    }
    uint32_t total = 0;
    bool anytie = false;
#pragma unroll
    for (int w = 0; w < WgScratch<NT>::W; ++w) {
      const uint32_t v = sh.red[bank][w];
      total = sat_add(total, v & 0x7fffffffu, kSat);
      anytie = anytie || (v >> 31);
    }
    bank ^= 1;
    if (!anytie && g.N + total < kGridTop) return grid_value(g.N + total, g.j);

    const uint32_t excl = wg_excl_scan_sat<NT>(tsum, kSat, sh, bank);
    uint32_t run = g.N + excl;
    uint32_t my_evt = 0xffffffffu;
    uint32_t my_before = 0;
    int my_k = 0;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int p = t * V + k;
      if (p > done && present(k) && my_evt == 0xffffffffu) {
        const uint32_t before = run;
        run += r[k];
        if (tie[k] || run >= kGridTop) {
          my_evt = (uint32_t)p;
          my_before = before;
          my_k = k;
        }
      }
    }
    const uint32_t P = wg_min_u32<NT>(my_evt, sh, bank);
    if (P == 0xffffffffu) return grid_value(g.N + total, g.j);
    const bool owner = my_evt == P;
    float s_post = 0.0f;
    uint32_t unused = 0;
    if (owner) s_post = grid_value(my_before, g.j) + E(my_k);
    wg_bcast<NT>(owner, s_post, unused, sh, bank);
    s = s_post;
    done = (int)P;
    if (done >= NT * V - 1) return s;
  }
}

// Accumulate term(p) for p in [0, len) in order, tile by tile (term may
// return -0.0f for an absent position).
template <int NT, int V, bool SUB, typename TermFn>
__device__ float list_accumulate(float s, int len, float thr, int& stop, TermFn term,
                                 WgScratch<NT>& sh, int& bank) {
  stop = -1;
  const int t = (int)threadIdx.x;
  for (int base = 0; base < len; base += NT * V) {
    float x[V];
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int p = base + t * V + k;
      x[k] = p < len ? term(p) : 0.0f;
    }
    int st;
    const int L = len - base < NT * V ? len - base : NT * V;
    s = tile_accumulate<NT, V, SUB>(s, x, L, thr, st, sh, bank);
    if (st >= 0) {
      stop = base + st;
      return s;
    }
  }
  return s;
}

}  // namespace llz
