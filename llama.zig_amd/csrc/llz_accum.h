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
// RN(term_k / 2^(j-23)) (saturated at kSat) and sets tie (a caller may also
// set tie to make an element an event when it cannot round it cheaply); E(k)
// returns the exact term, and is called only for an element at which an event
// is resolved; present(k) is false for positions outside the sequence.  Tile
// positions up to `done` are taken as already summed into s.  Lets a caller
// supply roundings from a cheaper, exact-when-unambiguous estimate.
//
// An event takes two barriers: the per-wave inclusive sums (with the tie
// flags) give every thread its exact prefix; each wave then resolves its own
// first event as if no earlier wave had one, and the first wave that has one
// holds the event (earlier waves' positions come first).
template <int NT, int V, typename RFn, typename EFn, typename PFn>
__device__ float tile_accumulate_fn(float s, RFn R, EFn E, PFn present, WgScratch<NT>& sh, int& bank,
                                    int done = -1) {
  constexpr int W = WgScratch<NT>::W;
  const int t = (int)threadIdx.x;
  const int w = wave_id();
  const int lane = lane_id();
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
    const uint32_t incl = wave_incl_scan_sat(tsum, kSat);
    const bool wt = bal64(ttie) != 0ull;
    if (lane == kWave - 1) sh.red[bank][w] = incl | (wt ? 0x80000000u : 0u);
    lds_barrier();
    uint32_t total = 0, before = 0;
    bool anytie = false;
#pragma unroll
    for (int i = 0; i < W; ++i) {
      const uint32_t v = sh.red[bank][i];
      total = sat_add(total, v & 0x7fffffffu, kSat);
      if (i < w) before = sat_add(before, v & 0x7fffffffu, kSat);
      anytie = anytie || (v >> 31);
    }
    if (!anytie && g.N + total < kGridTop) {
      bank ^= 1;
      return grid_value(g.N + total, g.j);
    }

    // this wave's first event, with the exact prefix before it
    uint32_t run = g.N + sat_add(before, wave_shift_up1(incl), kSat);
    int my_k = -1;
    uint32_t my_before = 0;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int p = t * V + k;
      if (p > done && present(k) && my_k < 0) {
        const uint32_t b = run;
        run += r[k];
        if (tie[k] || run >= kGridTop) {
          my_k = k;
          my_before = b;
        }
      }
    }
    const uint64_t em = bal64(my_k >= 0);
    const int owner = em != 0ull ? __ffsll((long long)em) - 1 : -1;
    if (lane == owner) {
      // E with a constant index (a caller's per-element arrays stay in registers)
      float x = 0.0f;
#pragma unroll
      for (int k = 0; k < V; ++k)
        if (k == my_k) x = E(k);
      sh.red[bank ^ 1][w] = (uint32_t)(t * V + my_k);
      sh.sw[w] = grid_value(my_before, g.j) + x;
    } else if (owner < 0 && lane == 0) {
      sh.red[bank ^ 1][w] = 0xffffffffu;
    }
    lds_barrier();
    uint32_t P = 0xffffffffu;
    float s_post = s;
#pragma unroll
    for (int i = 0; i < W; ++i) {
      const uint32_t q = sh.red[bank ^ 1][i];
      if (P == 0xffffffffu && q != 0xffffffffu) {
        P = q;
        s_post = sh.sw[i];
      }
    }
    // both banks were used: the next writer of red[bank] follows the second
    // barrier, after every read of it
    if (P == 0xffffffffu) return grid_value(g.N + total, g.j);  // unreachable
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
