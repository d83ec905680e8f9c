// llz_select.h -- the selection stage of the sampling chain (sampler.zig:89-168):
// candidate sort by (p desc, id asc), top-k / top-p / min-p, typical-p,
// total and the draw, with the streaming normaliser and a full-row radix
// sort as the fallbacks.  Included by the fused per-row kernel only.
#pragma once

#include "llz_accum.h"
#include "llz_bucket.h"
#include "llz_rowops.h"

namespace llz {

// Shared memory of the selection stage.
struct PostShared {
  uint64_t aux[kCap];       // (dev bits, id) for typical-p
  uint32_t aux_pos[kCap];   // p-order position carried through the dev sort
  uint8_t keep[kCap];       // final keep flag per p-order position
  RadixScratch radix;
};

struct SampleShared {
  WgScratch<kNT> wg;
  uint32_t cand_count;
  uint32_t misc[4];
  uint64_t cand[kCap];      // (e bits, id) while collecting, then (~p bits, id) sorted
  union {
    NormShared<kNT> norm;   // streaming normaliser (rows k_stats could not certify)
    PostShared post;        // sort, filters and draw
    BucketShared bkt;       // long kept prefixes without typical-p (llz_bucket.h)
  } u;
};

// Candidate list push (e >= theta): (e bits, id), capacity kCap.
__device__ __forceinline__ void push_candidate(SampleShared& sh, float e, uint32_t id) {
  const uint32_t slot = atomicAdd(&sh.cand_count, 1u);
  if (slot < (uint32_t)kCap) sh.cand[slot] = ((uint64_t)__float_as_uint(e) << 32) | id;
}

// Per-element state of a wave's slice for one base grid jb: wv holds the
// estimate q = e / 2^(jb-23), or, for special elements (bit set in spec),
// the exact term e.  Specials are the elements whose rounding is ambiguous
// in grid jb or jb+1, the large terms, and the candidates, so any rounding in
// those two grids follows from the state without a new exp.
struct SliceState {
  float wv[kSub][kV];
  uint32_t spec;   // bit c*kV + k
};

// RN(element / 2^(jj-23)) for jj in {jb, jb+1}; jj = jb + sh (sh = 0 or 1).
__device__ __forceinline__ uint32_t state_round(float w, bool spec, int jj, int sh, bool& tie) {
  tie = false;
  if (spec) return grid_round(w, jj, tie);
  return (uint32_t)rintf(fminf(sh ? w * 0.5f : w, 32768.0f));
}

// Sub-chunk sums (c >= c_from) in grid jb + sh from the slice state.
__device__ __forceinline__ void slice_sums(const SliceState& S, int sb, int n, int jb, int sh, int c_from,
                                           uint32_t* part) {
  const int lane = lane_id();
  uint32_t acc[kSub], tie_c = 0;
#pragma unroll
  for (int c = 0; c < kSub; ++c) {
    acc[c] = 0;
#pragma unroll
    for (int k = 0; k < kV; ++k) {
      const int p = sb + c * (kWave * kV) + lane * kV + k;
      if (c >= c_from && p < n) {
        bool tie;
        acc[c] = sat_add(acc[c], state_round(S.wv[c][k], (S.spec >> (c * kV + k)) & 1u, jb + sh, sh, tie), kSat);
        if (tie) tie_c |= 1u << c;
      }
    }
  }
  uint32_t sums[kSub];
#pragma unroll
  for (int c = 0; c < kSub; ++c) sums[c] = c < c_from ? 0u : wave_sum_sat(acc[c], kSat);
  uint32_t tie_w = 0;
#pragma unroll
  for (int c = 0; c < kSub; ++c) tie_w |= (bal64((tie_c >> c) & 1u) != 0ull) ? (1u << c) : 0u;
  if (lane == 0) {
#pragma unroll
    for (int c = 0; c < kSub; ++c)
      if (c >= c_from) part[c] = sums[c] | (((tie_w >> c) & 1u) ? 0x80000000u : 0u);
  }
}

// Slice state for base grid jb (sub-chunks c >= c_from), candidates on the
// first pass.  Exact terms of specials come from a per-wave queue so one
// rolled loop evaluates them densely.
__device__ __forceinline__ void slice_state(const float (&v)[kSub][kV], int sb, int n, float m, const RowParams& P,
                                            bool t1, int jb, bool first_pass, int c_from, SampleShared& sh,
                                            SliceState& S) {
  NormShared<kNT>& ns = sh.u.norm;
  const int lane = lane_id(), w = wave_id();
  const bool exact_mode = jb < -40;
  const float cj = (float)(23 - jb);
  const float qc = (exact_mode || !first_pass) ? (first_pass ? 0.0f : kInf)
                                               : ldexpf(P.cand_theta, 23 - jb) * (1.0f - 0x1p-14f);
  S.spec = 0;
#pragma unroll
  for (int c = 0; c < kSub; ++c) {
#pragma unroll
    for (int k = 0; k < kV; ++k) {
      const int p = sb + c * (kWave * kV) + lane * kV + k;
      const float q = __builtin_amdgcn_exp2f(fmaf(v[c][k] - m, P.l2e_t, cj));
      S.wv[c][k] = q;
      // ambiguous in grid jb or jb+1 (NaN-safe), large, or a candidate
      const float r0 = rintf(fminf(q, 32768.0f));
      const float h = q * 0.5f;
      const float r1 = rintf(fminf(h, 32768.0f));
      const bool amb = !(fmaf(q, kEps, fabsf(q - r0)) < 0.5f) || !(fmaf(h, kEps, fabsf(h - r1)) < 0.5f);
      const bool spec = c >= c_from && p < n && (exact_mode || amb || q >= qc);
      if (spec) S.spec |= 1u << (c * kV + k);
    }
  }
  if (bal64(S.spec != 0) == 0ull) return;
  const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
  int qn = 0;
#pragma unroll
  for (int e = 0; e < kSub * kV; ++e) {
    const bool sp = (S.spec >> e) & 1u;
    const uint64_t mk = bal64(sp);
    if (sp) {
      ns.ev[w][e][lane] = v[e / kV][e % kV];
      const int slot = qn + (int)__popcll(mk & lt);
      if (slot < kQCap) ns.q[w][slot] = (uint16_t)(e * kWave + lane);
    }
    qn += (int)__popcll(mk);
  }
  __builtin_amdgcn_wave_barrier();
  if (qn <= kQCap) {
    for (int i = lane; i < qn; i += kWave) {
      const uint32_t slot = ns.q[w][i];
      const uint32_t el = slot / kWave, ln = slot % kWave;
      const float x = exact_term(ns.ev[w][el][ln], m, P.temperature, t1);
      ns.ev[w][el][ln] = x;
      if (first_pass && x >= P.cand_theta)
        push_candidate(sh, x, (uint32_t)(sb + (int)(el / kV) * (kWave * kV) + (int)ln * kV + (int)(el % kV)));
    }
  } else {
    // more specials than the queue holds: each lane walks its own slots
    for (int el = 0; el < kSub * kV; ++el) {
      if ((S.spec >> el) & 1u) {
        const float x = exact_term(ns.ev[w][el][lane], m, P.temperature, t1);
        ns.ev[w][el][lane] = x;
        if (first_pass && x >= P.cand_theta)
          push_candidate(sh, x, (uint32_t)(sb + (el / kV) * (kWave * kV) + lane * kV + (el % kV)));
      }
    }
  }
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int e = 0; e < kSub * kV; ++e)
    if ((S.spec >> e) & 1u) S.wv[e / kV][e % kV] = ns.ev[w][e][lane];
  __builtin_amdgcn_wave_barrier();
}

// The exact running sum across sub-chunk oc of this wave's slice, by the
// owner wave, from the slice state.  Returns false (and leaves s at the
// last exact value, `done` at the last position consumed) when the sum
// leaves grids {jb, jb+1}: the caller then rebuilds the state.
__device__ __forceinline__ bool wave_resolve(float& s, int& done, const SliceState& S, const float (&v)[kSub][kV],
                                             int oc, int sb, int n, float m, const RowParams& P, bool t1, int jb) {
  const int lane = lane_id();
  const int base = sb + oc * (kWave * kV);
  float w4[kV], v4[kV];
  uint32_t sp4 = 0;
#pragma unroll
  for (int k = 0; k < kV; ++k) {
    w4[k] = 0.0f;
    v4[k] = 0.0f;
  }
#pragma unroll
  for (int c = 0; c < kSub; ++c)
    if (c == oc) {
#pragma unroll
      for (int k = 0; k < kV; ++k) {
        w4[k] = S.wv[c][k];
        v4[k] = v[c][k];
      }
      sp4 = (S.spec >> (c * kV)) & 0xfu;
    }
  for (;;) {
    const Grid g = grid_of(s);
    if (g.j != jb && g.j != jb + 1) return false;
    const int sh = g.j - jb;
    uint32_t r[kV];
    bool tie[kV];
    uint32_t tsum = 0;
#pragma unroll
    for (int k = 0; k < kV; ++k) {
      const int p = lane * kV + k;
      r[k] = 0;
      tie[k] = false;
      if (p > done && base + p < n) r[k] = state_round(w4[k], (sp4 >> k) & 1u, g.j, sh, tie[k]);
      tsum = sat_add(tsum, r[k], kSat);
    }
    const uint32_t incl = wave_incl_scan_sat(tsum, kSat);
    uint32_t run = g.N + wave_shift_up1(incl);
    int my_evt = -1, my_k = 0;
    uint32_t my_before = 0;
#pragma unroll
    for (int k = 0; k < kV; ++k) {
      const int p = lane * kV + k;
      if (my_evt < 0 && p > done && base + p < n) {
        const uint32_t before = run;
        run += r[k];
        if (tie[k] || run >= kGridTop) {
          my_evt = p;
          my_before = before;
          my_k = k;
        }
      }
    }
    const uint64_t mask = bal64(my_evt >= 0);
    if (mask == 0ull) {
      s = grid_value(g.N + lane_readlast(incl), g.j);
      done = kWave * kV - 1;
      return true;
    }
    const int L = __ffsll((long long)mask) - 1;
    const int kk = (int)readlane_u32((uint32_t)my_k, L);
    float wsel = 0.0f, vsel = 0.0f;
    bool ssel = false;
#pragma unroll
    for (int k = 0; k < kV; ++k)
      if (k == kk) {
        wsel = w4[k];
        vsel = v4[k];
        ssel = (sp4 >> k) & 1u;
      }
    const float ws = readlane_f32(wsel, L);
    const bool ss = readlane_u32(ssel ? 1u : 0u, L) != 0u;
    const float e = ss ? ws : exact_term(readlane_f32(vsel, L), m, P.temperature, t1);
    s = grid_value(readlane_u32(my_before, L), g.j) + e;
    done = (int)readlane_u32((uint32_t)my_evt, L);
    if (done >= kWave * kV - 1) return true;
  }
}

// sampler.zig:83-88: the exact sequential f32 normaliser of one row, plus the
// candidate list (every element with e >= cand_theta).
template <class Src>
__device__ float row_normaliser(const Src& X, int n, const RowParams& P, SampleShared& sh, int& bank,
                                float& m_out, float m_known) {
  constexpr int W = kNT / kWave;
  constexpr int GE = W * kSlice;    // elements per group
  constexpr int NC = W * kSub;      // sub-chunks per group
  static_assert(NC <= kWave, "one wave scans a group's sub-chunk sums");
  NormShared<kNT>& ns = sh.u.norm;
  const int lane = lane_id(), w = wave_id();
  const bool t1 = (P.flags & kFlagTIsOne) != 0;
  const bool vec = (P.flags & kFlagVecSrc) != 0;
  const int p0 = min(n, kPrologue);

  // independent loads first: the max partials, the prologue's logits and the
  // first group
  const float mp = m_known;
  const float vp = (w == 0 && lane < p0) ? X.at(lane) : 0.0f;
  float vcur[kSub][kV], vnext[kSub][kV];
#pragma unroll
  for (int c = 0; c < kSub; ++c) X.load4(p0 + w * kSlice + c * (kWave * kV) + lane * kV, n, vec, vcur[c]);
  const float m = wg_fmax<kNT>(mp, sh.wg, bank);
  m_out = m;

  // ---- prologue: the event-dense start of the row, the reference's loop
  if (w == 0) {
    float e = -0.0f;
    if (lane < p0) {
      e = exact_term(vp, m, P.temperature, t1);
      if (e >= P.cand_theta) push_candidate(sh, e, (uint32_t)lane);
    }
    float s0 = 0.0f;
    for (int l = 0; l < p0; ++l) s0 = s0 + readlane_f32(e, l);
    if (lane == 0) ns.s_bcast[0] = s0;
  }
  lds_barrier();
  float s = ns.s_bcast[0];
  int sbi = 1;
  int pb = 0;
  SliceState S;

  for (int gb = p0; gb < n; gb += GE) {
    if (gb + GE < n) {
#pragma unroll
      for (int c = 0; c < kSub; ++c)
        X.load4(gb + GE + w * kSlice + c * (kWave * kV) + lane * kV, n, vec, vnext[c]);
    }
    uint32_t* part = ns.part[pb];
    const int sb = gb + w * kSlice;
    int c0 = 0;        // first sub-chunk not yet added
    int dn = -1;       // positions of sub-chunk c0 already added (resolution in progress)
    // once the list has overflowed (the selection then reads the whole row
    // and never the list), candidates stop being special: their roundings
    // come from the estimates like every other element's (a wave reading
    // the count while others still push sees a smaller count at worst)
    bool first = __builtin_amdgcn_readfirstlane((int)sh.cand_count) <= kCap;
    for (;;) {  // (re)build the state for the grid of s
      const int jb = grid_of(s).j;
      slice_state(vcur, sb, n, m, P, t1, jb, first, max(0, c0 - w * kSub), sh, S);
      first = false;
      slice_sums(S, sb, n, jb, 0, max(0, c0 - w * kSub), &part[w * kSub]);
      lds_barrier();
      int j = jb;
      bool rebuilt = false;
      for (;;) {
        uint32_t N = grid_of(s).N;
        int cs;
        uint32_t before;
        if (dn >= 0) {
          // a resolution stopped inside sub-chunk c0: continue it there
          cs = c0;
          before = N;
        } else {
          const bool act = lane >= c0 && lane < NC;
          const uint32_t pv = act ? part[lane] : 0u;
          const uint32_t psum = pv & 0x7fffffffu;
          const uint32_t incl = wave_incl_scan_sat(psum, kSat);
          const uint32_t excl = wave_shift_up1(incl);
          const bool evt = act && ((pv >> 31) || g_top_reached(N, incl));
          const uint64_t mask = bal64(evt);
          if (mask == 0ull) {
            s = grid_value(N + lane_readlast(incl), j);
            c0 = NC;
            break;
          }
          cs = __ffsll((long long)mask) - 1;
          before = N + readlane_u32(excl, cs);
        }
        // resolve sub-chunk cs in its owner wave
        const int ow = cs / kSub, oc = cs % kSub;
        if (w == ow) {
          float so = grid_value(before, j);
          int d = dn;
          const bool ok = wave_resolve(so, d, S, vcur, oc, sb, n, m, P, t1, jb);
          if (lane == 0) {
            ns.s_bcast[sbi] = so;
            ns.part[pb ^ 1][NC] = ok ? 0xffffffffu : (uint32_t)d;  // resolution status
          }
        }
        lds_barrier();
        s = ns.s_bcast[sbi];
        sbi ^= 1;
        const uint32_t st = ns.part[pb ^ 1][NC];
        lds_barrier();
        if (st != 0xffffffffu) {
          // the sum left grids {jb, jb+1} inside sub-chunk cs: rebuild
          c0 = cs;
          dn = (int)st;
          rebuilt = true;
          break;
        }
        dn = -1;
        c0 = cs + 1;
        if (c0 >= NC) break;
        const int jn = grid_of(s).j;
        if (jn == j) continue;
        if (jn == jb + 1) {
          j = jn;
          if (w * kSub + kSub > c0) slice_sums(S, sb, n, jb, 1, max(0, c0 - w * kSub), &part[w * kSub]);
          lds_barrier();
          continue;
        }
        rebuilt = true;  // beyond jb+1: rebuild the state for the new grid
        break;
      }
      if (!rebuilt || c0 >= NC) break;
    }
    pb ^= 1;
#pragma unroll
    for (int c = 0; c < kSub; ++c)
#pragma unroll
      for (int k = 0; k < kV; ++k) vcur[c][k] = vnext[c][k];
  }
  return s;
}

// Sequential accumulation dispatcher: short lists run the reference's loop
// on one wave; long ones use the workgroup's exact parallel scan.
constexpr int kSeqMax = 128;

template <bool SUB, typename TermFn>
__device__ float seq_accumulate(float s, int len, float thr, int& stop, TermFn term, SampleShared& sh,
                                int& bank) {
  if (len <= kSeqMax) {
    float res = 0.0f;
    int st = -1;
    if (wave_id() == 0) res = wave_seq_list<SUB>(s, len, thr, st, term);
    uint32_t stu = (uint32_t)st;
    wg_bcast<kNT>(threadIdx.x == 0, res, stu, sh.wg, bank);
    stop = (int)stu;
    return res;
  }
  return list_accumulate<kNT, 2, SUB>(s, len, thr, stop, term, sh.wg, bank);
}

// Bitonic sort of u64 keys with a u32 payload, ascending.
template <int NT>
__device__ void lds_bitonic_sort_kv(uint64_t* a, uint32_t* pl, int n) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = (int)threadIdx.x; i < n; i += NT) {
        const int p = i ^ j;
        if (p > i) {
          const uint64_t x = a[i], y = a[p];
          const bool up = (i & k) == 0;
          if ((x > y) == up) {
            a[i] = y; a[p] = x;
            const uint32_t t = pl[i]; pl[i] = pl[p]; pl[p] = t;
          }
        }
      }
      lds_barrier();
    }
  }
}

__device__ __forceinline__ int next_pow2(int v) {
  int p = 2;
  while (p < v) p <<= 1;
  return p;
}

// Sorted-list views used by the filter stage: position q in (p desc, id asc).
struct LdsList {
  const uint64_t* a;
  __device__ float p(int q) const { return __uint_as_float(~(uint32_t)(a[q] >> 32)); }
  __device__ uint32_t id(int q) const { return (uint32_t)a[q]; }
};
struct GlobalList {
  const uint32_t* key;  // ~p bits
  const uint32_t* val;  // id
  __device__ float p(int q) const { return __uint_as_float(~key[q]); }
  __device__ uint32_t id(int q) const { return val[q]; }
};

// top-k / top-p / min-p over a sorted list whose first M positions are
// exactly the first M positions of the full order (sampler.zig:106-126).
// p_nc bounds the probability of every element beyond M (+inf when no bound
// is known).  Returns K (the kept prefix length) or -1 when positions beyond
// M decide.
// All three filters keep a prefix of the order, so the kept prefix length is
// min(Kk, Kp, Km); top-p's cut only matters when it falls before the other
// two, which is why min-p is resolved first.
template <typename List>
__device__ int prefix_filters(const List& L, int M, float p_nc, int n, const RowParams& P, float S,
                              SampleShared& sh, int& bank) {
  const int Kk = (P.top_k > 0 && P.top_k < (uint32_t)n) ? (int)P.top_k : n;
  int Km = n;  // n also stands for "at least M" when km_known is false
  bool km_known = true;
  if (P.min_p > 0.0f) {
    // probs[indices[0]] is the row maximum, e = exp(0) = 1, so p0 = 1/S
    const float p0 = 1.0f / S;
    const float thr = p0 * P.min_p;
    uint32_t cnt = 0;
    for (int q = (int)threadIdx.x; q < M; q += kNT) cnt += L.p(q) >= thr ? 1u : 0u;
    cnt = wg_sum_sat<kNT>(cnt, 0x7fffffffu, sh.wg, bank);
    if ((int)cnt < M) Km = (int)cnt;
    else if (M < n) {
      if (thr > p_nc) Km = M;
      else km_known = false;
    }
  }
  int Kp = n;
  if (P.top_p > 0.0f && P.top_p < 1.0f) {
    const int bound = min(Kk, Km);
    const int lim = min(bound, M);
    int st;
    seq_accumulate<false>(0.0f, lim, P.top_p, st, [&](int q) { return L.p(q); }, sh, bank);
    if (st >= 0) Kp = st;
    else if (bound > M) return -1;  // the cut may lie beyond the certified prefix
  }
  (void)km_known;  // an unknown Km >= M only matters if the result exceeds M
  const int K = min(Kk, min(Kp, Km));
  return K > M ? -1 : K;
}

// A row read tile by tile, V logits per thread (thread t holds positions
// t*V .. t*V+V-1 of a tile of 512 V), with the next tile's loads issued
// before the current tile's work.  With 16-byte loads every thread loads
// from min(pos, nlast) (the last start that stays inside the row), so no
// branch separates a tile's loads from the work they overlap; the one
// thread whose span crosses the row's end re-reads its logits where they are
// used (fix_tail).  Positions past the row read as 0.
template <int V_>
struct RowTilesT {
  static constexpr int V = V_;
  static_assert(V % 4 == 0, "whole float4 per thread");
  const float* xs;
  int n;
  bool vec8;
  int nlast;
  __device__ RowTilesT(const float* x, int n_, bool vec) : xs(x), n(n_), vec8(vec && n_ >= V),
                                                          nlast(vec && n_ >= V ? ((n_ - V) & ~3) : 0) {}
  // the row through a global-address-space pointer: the callers run out of
  // line, where a generic pointer would make these flat loads, which count
  // on the LDS counter too (every LDS wait would wait for them)
  __device__ __forceinline__ const __attribute__((address_space(1))) float* g() const {
    return (const __attribute__((address_space(1))) float*)xs;
  }
  __device__ __forceinline__ void load(int pos, float (&r)[V]) const {
    if (vec8) {
      const int pc = min(pos, nlast);
#pragma unroll
      for (int h = 0; h < V / 4; ++h) {
        const llz_f4v q = *(const __attribute__((address_space(1))) llz_f4v*)(g() + pc + 4 * h);
        r[4 * h + 0] = q.x; r[4 * h + 1] = q.y; r[4 * h + 2] = q.z; r[4 * h + 3] = q.w;
      }
    } else {
#pragma unroll
      for (int k = 0; k < V; ++k) r[k] = pos + k < n ? g()[pos + k] : 0.0f;
    }
  }
  __device__ __forceinline__ void fix_tail(int pos, float (&r)[V]) const {
    if (vec8 && pos > nlast && pos < n) {
#pragma unroll
      for (int k = 0; k < V; ++k) r[k] = pos + k < n ? g()[pos + k] : 0.0f;
    }
  }
};
using RowTiles8 = RowTilesT<8>;

// Entropy sum over the whole row in index order (sampler.zig:129-132):
// entropy -= p * log(p) for every p = RN(e / S) > 0, which is the exact
// sequential sum of the terms t = -RN(p * log(p)) >= 0 (a - b == a + (-b)).
// Wave 0 sums the first 512 terms alone (wave_accumulate: the many binade
// crossings of a sum that starts at 0 cost no barriers there); the rest goes
// through tile_accumulate_fn, which needs of each term its rounding RN(t / u)
// on the running sum's grid u = 2^(j-23), taken from an estimate wherever the
// estimate's error bound fixes it.
//
// Estimate, for 2^-110 <= p~ <= 2^-2, from the reference's own argument x =
// RN(RN(v - m) / T):
//   x log2(e) = a_hi + a_lo (a_hi = RN(x L2E), a_lo = fma(x, L2E, -a_hi) +
//   x L2E_lo, L2E + L2E_lo = log2(e) to 2^-49);  e~ = fma(e0, a_lo ln2, e0),
//   e0 = exp2(a_hi);  p~ = RN(e~ RN(1 / S));  l~ = RN(log2(p~) RN(ln 2));
//   t~ = -RN(p~ l~).
// Relative errors against the reference's e = expf(x) (< 1 ulp), p = RN(e /
// S), l = logf(p) (< 1 ulp), t: the hardware exp2 and log2 are taken to be
// within 1 ulp of their results; e~ / exp(x) - 1 <= 1.5 * 2^-23 (exp2, the
// fma, and terms below 2^-33); p~ / p - 1 <= dp = 4 * 2^-23; with |log p| >=
// ln 4, l~ / l - 1 <= dp / ln 4 + 3 * 2^-23; so t~ / t - 1 <= 10.9 * 2^-23 to
// first order, and eps = 24 * 2^-23 is more than twice that.  y~ = t~
// 2^(23-j) is exact; when [y~(1 - eps), y~(1 + eps)] lies strictly between k
// - 1/2 and k + 1/2 (y~ < 2^22), RN(t / u) = k and t / u is no tie; when y~(1
// - eps) >= 2^24 the term leaves the binade by itself (kSat, as grid_round).
// Below: p~ < 2^-110 (or x < -88) means p < 2^-108, so t < 2^-108 * 88 <
// 2^-101.5 rounds to 0 on every grid j >= -60.  NaN estimates, p~ > 2^-2,
// finer grids and uncertain roundings take the exact term, evaluated once per
// element with the reference's operations.
// Out of line, so that the kernel's common path does not carry its
// registers; the row's parameters come by value (a reference would make the
// kernel store them to its stack).

struct EntropyResult {
  float H;
  int bank;
};

template <class Src>
__device__ __noinline__ EntropyResult entropy_pass(Src X, int n, float m, float S, float T, uint32_t flags,
                                                   SampleShared& sh_arg, int bank, int row) {
  // Out of line, the function receives generic pointers: the shared memory
  // recast to the LDS address space (RowTiles8 reads the row through a
  // global one), so that the accesses are ds_ and global_ instructions.  A
  // flat access counts on both the LDS and the vector memory counters, so
  // each LDS wait would also wait for the next tile's loads in flight.
  SampleShared& sh = *(SampleShared*)(__attribute__((address_space(3))) SampleShared*)(&sh_arg);
  constexpr int EV = 2 * kLaneV;  // logits per thread per tile
  constexpr int ET = kNT * EV;
  constexpr int EP = kWave * EV;  // the prologue's terms (wave 0's share of the first tile)
  constexpr float L2E = 1.44269502e+0f;     // RN(log2(e))
  constexpr float L2E_LO = 1.92596303e-8f;  // RN(log2(e) - L2E)
  constexpr float LN2 = 6.93147182e-1f;     // RN(ln 2)
  constexpr float EPS = 24.0f * 0x1p-23f;
  const bool t1 = (flags & kFlagTIsOne) != 0;
  const bool vec = (flags & kFlagVecSrc) != 0;
  const float rS = 1.0f / S;
  const int t = (int)threadIdx.x;

  const RowTilesT<EV> rt(X.x, n, vec);
  // sampler.zig:85 and :131 on one argument x; the term is +0 when p == 0
  auto exact_term = [&](float x) {
    const float p = exp_f32(x) / S;
    return p > 0.0f ? -(p * log_f32(p)) : 0.0f;
  };

  float raw[EV];
  rt.load(t * EV, raw);
  rt.fix_tail(t * EV, raw);
  float H = 0.0f;
  {
    uint32_t unused = 0;
    if (wave_id() == 0) {
      float x[EV];
#pragma unroll
      for (int k = 0; k < EV; ++k) {
        const int pos = t * EV + k;
        float a = X.fix(pos, raw[k]) - m;
        if (!t1) a = a / T;
        const float te = exact_term(a);
        x[k] = pos < n && te > 0.0f ? te : -0.0f;  // absent: past the row, or p * log(p) == 0
      }
      H = wave_accumulate<EV>(0.0f, x);
    }
    wg_bcast<kNT>(t == 0, H, unused, sh.wg, bank);
  }
  LLZ_STAMP(row, 48);

  for (int base = 0; base < n; base += ET) {
    const int pos = base + t * EV;
    if (base == 20 * ET) LLZ_STAMP(row, 53);
    if (base > 0) rt.fix_tail(pos, raw);
    float xa[EV];
#pragma unroll
    for (int k = 0; k < EV; ++k) {
      float a = (pos + k < n ? X.fix(pos + k, raw[k]) : 0.0f) - m;
      if (!t1) a = a / T;
      xa[k] = a;  // the reference's argument
    }
    if (base + ET < n) rt.load(pos + ET, raw);  // the next tile's loads fly during this one

    float tl[EV], te[EV];
    uint32_t mid = 0, tiny = 0, have = 0;
#pragma unroll
    for (int k = 0; k < EV; ++k) {
      const float x = xa[k];
      const float ah = x * L2E;
      const float al = fmaf(x, L2E, -ah) + x * L2E_LO;
      const float e0 = __builtin_amdgcn_exp2f(ah);
      const float pt = fmaf(e0, al * LN2, e0) * rS;
      tl[k] = -(pt * (__builtin_amdgcn_logf(pt) * LN2));
      te[k] = 0.0f;
      const bool tn = x < -88.0f || pt < 0x1p-110f;
      tiny |= (tn ? 1u : 0u) << k;
      mid |= (!tn && pt <= 0x1p-2f ? 1u : 0u) << k;
    }
    auto exact = [&](int k) {
      if (!((have >> k) & 1u)) {
        // the empty volatile asm keeps the evaluation inside this branch:
        // the term is loop-invariant in tile_accumulate_fn, and hoisted out
        // of the branch it would be computed for every element
        float x = xa[k];
        asm volatile("" : "+v"(x));
        te[k] = exact_term(x);
        have |= 1u << k;
      }
      return te[k];
    };
    // the rounding on grid j from the estimate: true when the estimate's
    // error bound fixes it (out), false when the exact term must decide
    auto cheap = [&](int k, int j, uint32_t& out) -> bool {
      const float y = ldexpf(tl[k], 23 - j);
      const float d = y * EPS;
      const float r = rintf(y);
      const bool big = y - d >= 0x1p24f;
      const bool cert = y < 0x1p22f && fabsf(y - r) + d < 0.5f;
      const bool is_tiny = ((tiny >> k) & 1u) != 0u;
      out = is_tiny ? 0u : (big ? kSat : (uint32_t)r);
      return is_tiny ? j >= -60 : (((mid >> k) & 1u) != 0u && (big || cert));
    };
    // the certified cases are selected without branches; one branch per
    // element leads to the exact term
    auto R = [&](int k, int j, bool& tie) -> uint32_t {
      tie = false;
      uint32_t out;
      if (!cheap(k, j, out)) out = grid_round(exact(k), j, tie);
      return out;
    };
    auto E = [&](int k) { return exact(k); };
    auto present = [&](int k) { return pos + k < n; };
    if (base == 20 * ET) LLZ_STAMP(row, 54);
    H = tile_accumulate_fn<kNT, EV>(H, R, E, present, sh.wg, bank, base == 0 ? EP - 1 : -1);
    if (base == 0) LLZ_STAMP(row, 49);
    if (base == ET) LLZ_STAMP(row, 50);
    if (base == 16 * ET) LLZ_STAMP(row, 51);
    if (base == 20 * ET) LLZ_STAMP(row, 55);
  }
  LLZ_STAMP(row, 52);
  return EntropyResult{H, bank};
}

// Total and draw over p-order positions [0, K) whose keep flag is set
// (sampler.zig:156-168).  keep(q) -> bool.
// first: the id of indices[0] (the row's first element in p order) when L
// does not start with it (0xffffffff: L.id(0)).
template <typename List, typename Keep>
__device__ void total_and_draw(const List& L, int K, Keep keep, float u, float& total,
                               uint32_t& token, uint32_t& consumed, SampleShared& sh, int& bank,
                               uint32_t first = 0xffffffffu) {
  int st;
  total = seq_accumulate<false>(0.0f, K, -1.0f, st, [&](int q) { return keep(q) ? L.p(q) : -0.0f; }, sh,
                                bank);
  const uint32_t tok0 = first != 0xffffffffu ? first : L.id(0);
  if (total <= 0.0f) {
    token = tok0;
    consumed = 0;
    return;
  }
  consumed = 1;
  const float r0 = u * total;
  seq_accumulate<true>(r0, K, -1.0f, st, [&](int q) { return keep(q) ? L.p(q) : -0.0f; }, sh, bank);
  token = st >= 0 ? L.id(st) : tok0;
}

// Rare paths of k_select, out of line so that the common path's register
// allocation stays small.

struct NormResult {
  float S, m;
  int bank;
};

// k_stats's argument (KArgs) where the kernel received it, in its argument
// segment: the out-of-line fallbacks read it through this pointer instead of
// from a copy in their stack frame (a copy the compiler stores in every
// launch's prologue).  The segment pointer exists in the kernel only (a
// callee's builtin yields null), so the kernel takes it and passes it down.
__device__ __forceinline__ const KArgs* kernel_args_ptr() {
  return (const KArgs*)__builtin_amdgcn_kernarg_segment_ptr();  // address-space cast to a generic pointer
}

// The chain's reader of row `row` for a reader type.
template <class Src>
__device__ __forceinline__ Src make_src(const RowParams& P, const RowPtrs& Q, int row, const PenShared* pen) {
  if constexpr (std::is_same<Src, RowSrc>::value) {
    return row_src<true>(P, Q, row, pen);
  } else if constexpr (std::is_same<Src, LightSrc>::value) {
    return row_src<false>(P, Q, row, pen);
  } else {
    return PlainSrc{Q.src + (int64_t)row * P.src_stride};
  }
}

// The streaming normaliser (sampler.zig:83-88) for a row k_stats could not
// certify; fills the candidate list in LDS.
template <class Src>
__device__ __noinline__ NormResult select_norm_fallback(const KArgs* A, int row, const PenShared* pen, SampleShared& sh,
                                                        int bank, float m_known) {
  const RowParams& P = A->P;
  const Src X = make_src<Src>(P, A->Q, row, pen);
  // the shared memory in the LDS address space (a generic reference would
  // make every access flat)
  SampleShared& shl = *(SampleShared*)(__attribute__((address_space(3))) SampleShared*)(&sh);
  if (threadIdx.x == 0) shl.cand_count = 0;
  NormResult r;
  r.S = row_normaliser(X, P.n, P, shl, bank, r.m, m_known);
  r.bank = bank;
  return r;
}

template <class Src>
__device__ __noinline__ void select_full_row(const KArgs* A, int row, const PenShared* pen, SampleShared& sh,
                                             int bank, float m, float S, uint32_t path);

constexpr int kShortMax = 256;  // longest candidate list of the short path

// A flooded candidate list (more than kCap elements with e >= cand_theta) is
// collected again from the row, keeping only its largest terms, so that the
// selection still runs on a list whenever the kept prefix is short: the
// reference's default chain (top-p 0.9, no min-p) on peaked rows keeps tens
// to hundreds of terms of the thousands above 2^-16.  e is monotone in v, so
// the largest terms are the largest logits:
//  1. a histogram of d = m - v over [0, D), D = T ln(1 / cand_theta) (1 +
//     2^-10) (every candidate), kRecBins bins of width w, with the count and
//     the estimated terms' sum of each;
//  2. the cut b: the first bin where the running estimated mass reaches
//     top_p S (1 + 2^-8) (the estimates are within 2^-16 of the terms), one
//     bin more, or else the end; and no further than the bins whose elements
//     fit the list with a quarter of it to spare;
//  3. every element with v > v_t = m - b w, with its exact term (sampler.zig:85).
// Every element left out has v <= v_t, so e <= e(v_t) (1 + 2^-21.9): the
// reference's argument RN(RN(v - m) / T) is monotone in v and its exp is
// within one ulp of exp.  Returns e(v_t) (1 + 2^-21), the bound the
// selection's certified prefix takes in place of cand_theta, or -1 when the
// list cannot be made to fit (the full-row fallback follows).
constexpr int kRecBins = 2048;

template <class Src>
__device__ __noinline__ float recollect_top(const Src X, int n, float m, float S, float T, float theta,
                                            float l2e_t, float top_p, uint32_t top_k, uint32_t flags,
                                            SampleShared& sh, int bank, int row) {
  constexpr int EV = RowTiles8::V;
  constexpr int ET = kNT * EV;
  constexpr int HB = kRecBins;
  static_assert(sizeof(sh.u.post.radix.stage_k) >= HB * sizeof(uint32_t), "histogram counts fit");
  static_assert(sizeof(sh.u.post.radix.stage_v) >= HB * sizeof(float), "histogram sums fit");
  uint32_t* hcnt = sh.u.post.radix.stage_k;
  float* hsum = reinterpret_cast<float*>(sh.u.post.radix.stage_v);
  const int t = (int)threadIdx.x;
  const bool t1 = (flags & kFlagTIsOne) != 0;
  const bool vec = (flags & kFlagVecSrc) != 0;
  // D: T ln(1/theta) from the hardware log2 (within an ulp), with 2^-10 to spare
  const float D = T * (-__builtin_amdgcn_logf(theta)) * 0.693147182f * (1.0f + 0x1p-10f);
  if (!(D > 0.0f) || !(D < 3.0e38f)) return -1.0f;
  const float w = D / (float)HB, iw = (float)HB / D;
  for (int b = t; b < HB; b += kNT) {
    hcnt[b] = 0u;
    hsum[b] = 0.0f;
  }
  lds_barrier();
  const RowTiles8 rt(X.x, n, vec);
  float raw[EV];
  // ---- 1. the histogram (d < D: NaN and -inf logits never enter)
  rt.load(t * EV, raw);
  for (int base = 0; base < n; base += ET) {
    const int pos = base + t * EV;
    rt.fix_tail(pos, raw);
    float d[EV];
#pragma unroll
    for (int k = 0; k < EV; ++k) d[k] = pos + k < n ? m - X.fix(pos + k, raw[k]) : kInf;
    if (base + ET < n) rt.load(pos + ET, raw);
#pragma unroll
    for (int k = 0; k < EV; ++k) {
      if (d[k] < D) {
        const int b = min(HB - 1, (int)(d[k] * iw));
        atomicAdd(&hcnt[b], 1u);
        atomicAdd(&hsum[b], __builtin_amdgcn_exp2f(-d[k] * l2e_t));
      }
    }
  }
  lds_barrier();
  LLZ_STAMP(row, 40);
  // ---- 2. the cut: wave 0, lane l holding bins 32 l .. 32 l + 31
  if (wave_id() == 0) {
    constexpr int PB = HB / kWave;
    const int lane = lane_id();
    uint32_t cnt_l = 0u;
    float mass_l = 0.0f;
    for (int j = 0; j < PB; ++j) {
      cnt_l += hcnt[lane * PB + j];
      mass_l += hsum[lane * PB + j];
    }
    const uint32_t cinc = wave_incl_scan_op(cnt_l, 0u, [](uint32_t a, uint32_t b) { return a + b; });
    const float minc = __uint_as_float(wave_incl_scan_op(__float_as_uint(mass_l), 0u, [](uint32_t a, uint32_t b) {
      return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
    }));
    const uint32_t cap_fit = (uint32_t)(kCap - kCap / 4);
    const bool topk_fit = top_k > 0u && top_k <= cap_fit / 2u;  // top-k ends the prefix inside a full list
    const bool topp = top_p > 0.0f && top_p < 1.0f;
    const float mass_target = topp ? top_p * S * (1.0f + 0x1p-8f) : kInf;
    // the first bin where the list would be full, and the first where the
    // running mass reaches top-p's target (then one bin more)
    uint32_t c = cinc - cnt_l;
    float s = minc - mass_l;
    int cut_full = HB, mass_bin = HB;
    for (int j = 0; j < PB; ++j) {
      const int b = lane * PB + j;
      c += hcnt[b];
      s += hsum[b];
      if (c > cap_fit && cut_full == HB) cut_full = b;  // bins before b fit the list
      if (s >= mass_target && mass_bin == HB) mass_bin = b;
    }
    const int full_at = (int)wave_min_u32((uint32_t)cut_full);
    const int mass_at = (int)wave_min_u32((uint32_t)mass_bin);
    // a list filled at or before the bin where top-p's mass is reached,
    // without a top-k inside it, cannot hold the kept prefix: not worth the
    // second pass
    const bool hopeless = full_at < HB && full_at <= mass_at && !topk_fit;
    if (lane == 0) sh.misc[2] = hopeless ? 0u : (uint32_t)min(full_at, min(HB, mass_at + 2));
  }
  lds_barrier();
  const int cut = (int)sh.misc[2];
  if (cut <= 0) return -1.0f;  // the top bin alone does not fit
  const float v_t = m - (float)cut * w;
  if (t == 0) sh.cand_count = 0u;
  lds_barrier();
  LLZ_STAMP(row, 41);
  // ---- 3. every element above v_t, with its exact term
  rt.load(t * EV, raw);
  for (int base = 0; base < n; base += ET) {
    const int pos = base + t * EV;
    rt.fix_tail(pos, raw);
    float v[EV];
#pragma unroll
    for (int k = 0; k < EV; ++k) v[k] = pos + k < n ? X.fix(pos + k, raw[k]) : -kInf;
    if (base + ET < n) rt.load(pos + ET, raw);
#pragma unroll
    for (int k = 0; k < EV; ++k)
      if (v[k] > v_t) push_candidate(sh, exact_term(v[k], m, T, t1), (uint32_t)(pos + k));
  }
  lds_barrier();
  LLZ_STAMP(row, 42);
  if (sh.cand_count > (uint32_t)kCap) return -1.0f;
  return exact_term(v_t, m, T, t1) * (1.0f + 0x1p-21f);
}

// The selection for a short candidate list without typical-p (the common
// case): a rank sort by every wave, then filters, total and draw by wave 0
// alone (sampler.zig:92-126, 156-168), with the same certified-prefix rules
// as prefix_filters.  Returns false, on every thread, when elements outside
// the list decide the cut: the caller then takes the full-row fallback.
__device__ __forceinline__ bool select_short(const RowParams& P, const RowPtrs& Q, int row, SampleShared& sh, int c,
                                             float m, float S, uint32_t path, float u_row) {
  const int t = (int)threadIdx.x, lane = lane_id(), w = wave_id();
  const int n = P.n;
  uint64_t* key = sh.cand;               // (~p bits, id): ascending = (p desc, id asc)
  uint32_t* rank = sh.u.post.aux_pos;
  uint64_t* srt = sh.u.post.aux;
  // probabilities as sampler.zig:90 computes them
  for (int i = t; i < c; i += kNT) {
    const uint64_t a = key[i];
    const float p = __uint_as_float((uint32_t)(a >> 32)) / S;
    key[i] = ((uint64_t)(~__float_as_uint(p)) << 32) | (uint32_t)a;
    rank[i] = 0;
  }
  lds_barrier();
  // rank = number of smaller keys (keys are distinct: the ids are); wave w
  // counts against its eighth of the list
  {
    constexpr int NW = kNT / kWave;
    const int j0 = (w * c) / NW, j1 = ((w + 1) * c) / NW;
    for (int i = lane; i < c; i += kWave) {
      const uint64_t ki = key[i];
      uint32_t r = 0;
      int j = j0;
      for (; j + 4 <= j1; j += 4) {  // four LDS reads in flight
        const uint64_t a0 = key[j], a1 = key[j + 1], a2 = key[j + 2], a3 = key[j + 3];
        r += (a0 < ki ? 1u : 0u) + (a1 < ki ? 1u : 0u) + (a2 < ki ? 1u : 0u) + (a3 < ki ? 1u : 0u);
      }
      for (; j < j1; ++j) r += key[j] < ki ? 1u : 0u;
      if (r != 0u) atomicAdd(&rank[i], r);
    }
  }
  lds_barrier();
  for (int i = t; i < c; i += kNT) srt[rank[i]] = key[i];
  lds_barrier();
  if (w == 0) {
    auto pq = [&](int q) { return __uint_as_float(~(uint32_t)(srt[q] >> 32)); };
    // the list's first 64 probabilities, one per lane, read once (xl; the
    // lanes past the list hold -0, an absent term): every chain over at most
    // 64 terms, and the counts over a list of at most 64, use them
    const float xl = lane < c ? pq(lane) : -0.0f;
    // certified prefix M: every element outside the list has p <= theta / S
    const float p_nc = P.cand_theta / S;
    int M = c;
    if (P.cand_theta > 0.0f) {
      M = 0;
      if (c <= kWave) M = __popcll(bal64(lane < c && xl > p_nc));
      else
        for (int b = 0; b < c; b += kWave) M += __popcll(bal64(b + lane < c && pq(b + lane) > p_nc));
    }
    // top-k, min-p, top-p (sampler.zig:106-126): each keeps a prefix
    const int Kk = (P.top_k > 0 && P.top_k < (uint32_t)n) ? (int)P.top_k : n;
    int Km = n;
    if (P.min_p > 0.0f) {
      const float thr = (1.0f / S) * P.min_p;  // probs[indices[0]] = 1 / S: the row maximum has e = 1
      int cnt = 0;
      if (M <= kWave) cnt = __popcll(bal64(lane < M && xl >= thr));
      else
        for (int b = 0; b < M; b += kWave) cnt += __popcll(bal64(b + lane < M && pq(b + lane) >= thr));
      if (cnt < M) Km = cnt;
      else if (M < n && thr > p_nc) Km = M;
    }
    int K = min(Kk, Km);
    bool undecided = false;
    // acc, lane i: the running sum from 0 after term i, over the first
    // `covered` terms (the top-p chain and the total add the same terms in
    // the same order from 0, so the total is a value of the same chain)
    float acc = 0.0f;
    int covered = 0;
    if (P.top_p > 0.0f && P.top_p < 1.0f) {
      const int lim = min(K, M);
      int st;
      if (lim <= kWave) {
        acc = wave_chain_lanes<false>(0.0f, xl, lim);
        covered = lim;
        const uint64_t hits = bal64(lane < lim && acc > P.top_p);
        st = hits != 0ull ? __ffsll((long long)hits) - 1 : -1;
      } else {
        wave_seq_list<false>(0.0f, lim, P.top_p, st, pq);
      }
      if (st >= 0) K = min(K, st);
      else if (K > M) undecided = true;
    }
    if (K > M) undecided = true;
    if (!undecided) {
      // total and draw (sampler.zig:156-168); K <= M <= c here
      int st;
      float total;
      if (K <= kWave) {
        if (covered < K) acc = wave_chain_lanes<false>(0.0f, xl, K);
        total = K > 0 ? readlane_f32(acc, K - 1) : 0.0f;
      } else {
        total = wave_seq_list<false>(0.0f, K, -1.0f, st, pq);
      }
      const uint32_t tok0 = (uint32_t)srt[0];
      uint32_t token = tok0, consumed = 0;
      if (total > 0.0f) {
        consumed = 1;
        if (K <= kWave) {
          const float r = wave_chain_lanes<true>(u_row * total, xl, K);
          const uint64_t hits = bal64(lane < K && r <= 0.0f);
          st = hits != 0ull ? __ffsll((long long)hits) - 1 : -1;
        } else {
          wave_seq_list<true>(u_row * total, K, -1.0f, st, pq);
        }
        if (st >= 0) token = (uint32_t)srt[st];
      }
      if (Q.kept_ids || Q.kept_probs) {
        for (int q = lane; q < K && q < P.kept_cap; q += kWave) {
          if (Q.kept_ids) Q.kept_ids[(int64_t)row * P.kept_cap + q] = (uint32_t)srt[q];
          if (Q.kept_probs) Q.kept_probs[(int64_t)row * P.kept_cap + q] = pq(q);
        }
      }
      if (lane == 0) {
        Q.tokens[row] = token;
        if (Q.consumed) Q.consumed[row] = (uint8_t)consumed;
        if (Q.kept_count) Q.kept_count[row] = (uint32_t)K;
        if (Q.row_stats) {
          float* rs = Q.row_stats + (int64_t)row * 4;
          rs[0] = m; rs[1] = S; rs[2] = 0.0f; rs[3] = total;
        }
        if (Q.status) Q.status[row] = path;
      }
    }
    if (lane == 0) sh.misc[0] = undecided ? 1u : 0u;
  }
  lds_barrier();
  return sh.misc[0] == 0u;
}

// The rest of sampleWithRandom (sampler.zig:89-168) for row `row`,
// after k_stats' phases: from the row maximum m, the normaliser S and the
// candidate list in Q.cand (cc entries), or, for a row k_stats could not
// certify, from the streaming normaliser.  Every thread of the workgroup
// calls it; `sh` may alias the caller's shared memory once all of it is read.
// pre_ok: thread 64 + i holds candidate i in cand_pre for i < cand_n0, and
// cc_in <= 448 (the later ones are read here).
template <class Src, class OSrc>
__device__ __forceinline__ void select_row(const RowParams& P, const RowPtrs& Q, SampleShared& sh, float m,
                                           float S, uint32_t cc_in, bool uncertified, float u_row, bool pre_ok,
                                           uint64_t cand_pre, uint32_t cand_n0, const Src& X, const OSrc& O,
                                           const PenShared* pen, const KArgs* A, int row) {
  int bank = 0;
  const int t = (int)threadIdx.x;
  const int n = P.n;
  uint32_t path = 0;
  if (uncertified) {
    // the streaming normaliser (sampler.zig:83-88) fills the candidate list in LDS
    const NormResult r = select_norm_fallback<Src>(A, row, pen, sh, bank, m);
    LLZ_STAMP(row, 7);
    S = r.S;
    m = r.m;
    bank = r.bank;
    path |= kPathNormFallback;
  } else {
    const int c = cc_in > (uint32_t)kCap ? kCap : (int)cc_in;
    if (pre_ok) {
      const int i = t - kWave;
      if (t >= kWave && i < c) sh.cand[i] = i < (int)cand_n0 ? cand_pre : Q.cand[(int64_t)row * kCap + i];
    } else {
      const uint64_t* gc = Q.cand + (int64_t)row * kCap;
      for (int i = t; i < c; i += kNT) sh.cand[i] = gc[i];
    }
    if (t == 0) sh.cand_count = cc_in;
  }
  uint32_t token = 0, consumed = 0;
  float H = 0.0f, total = 0.0f;
  int K = 0;

  // ---- 3. sum <= 0 exit: sampleArgmax of the caller's logits (:89)
  if (S <= 0.0f) {
    token = wg_argmax_row<kNT>(O, n, sh.wg, bank);
    path = kPathSumLe0;
    if (t == 0) {
      Q.tokens[row] = token;
      if (Q.consumed) Q.consumed[row] = 0;
      if (Q.kept_count) Q.kept_count[row] = 0;
      if (Q.row_stats) {
        float* rs = Q.row_stats + (int64_t)row * 4;
        rs[0] = m; rs[1] = S; rs[2] = 0.0f; rs[3] = 0.0f;
      }
      if (Q.status) Q.status[row] = path;
    }
    return;
  }

  // ---- a NaN normaliser (a NaN logit or an infinite maximum): every
  // probability is NaN, so every comparison of the chain is false.  The
  // stable sort keeps index order, top-k keeps the first k indices, top-p,
  // min-p and typical-p keep everything, the total is NaN and the walk never
  // stops: indices[0] = 0 after one draw (sampler.zig:96-168).
  if (S != S) {
    const int kept = (P.top_k > 0 && P.top_k < (uint32_t)n) ? (int)P.top_k : n;
    if (Q.kept_ids || Q.kept_probs) {
      for (int q = t; q < kept && q < P.kept_cap; q += kNT) {
        if (Q.kept_ids) Q.kept_ids[(int64_t)row * P.kept_cap + q] = (uint32_t)q;
        if (Q.kept_probs) Q.kept_probs[(int64_t)row * P.kept_cap + q] = __builtin_nanf("");
      }
    }
    if (t == 0) {
      Q.tokens[row] = 0;
      if (Q.consumed) Q.consumed[row] = 1;
      if (Q.kept_count) Q.kept_count[row] = (uint32_t)kept;
      if (Q.row_stats) {
        float* rs = Q.row_stats + (int64_t)row * 4;
        rs[0] = m; rs[1] = S; rs[2] = 0.0f; rs[3] = __builtin_nanf("");
      }
      if (Q.status) Q.status[row] = 0;
    }
    return;
  }

  // ---- 4. candidates -> probabilities -> (p desc, id asc) (:90-100)
  lds_barrier();
  uint32_t cc = sh.cand_count;
  // the list's threshold for the certified prefix: cand_theta, or the bound
  // of a list collected again (recollect_top) after it flooded
  RowParams Pl = P;
  // only where a filter can end the kept prefix inside the list: top-p, or a
  // top-k within three quarters of it (min-p alone keeps every flooded term)
  const bool bounded = (P.top_p > 0.0f && P.top_p < 1.0f) || (P.top_k > 0u && P.top_k <= (uint32_t)(kCap - kCap / 4) / 2u);
  // (each term is at most 1, so a kept prefix that top-p alone ends inside
  // the list needs top_p S <= the list's length: near-flat rows skip it)
  const bool topk_in = P.top_k > 0u && P.top_k <= (uint32_t)(kCap - kCap / 4) / 2u;
  const bool reachable = topk_in || P.top_p * S <= (float)(kCap - kCap / 4);
  if (cc > (uint32_t)kCap && n > kCap && P.cand_theta > 0.0f && bounded && reachable) {
    const float th =
        recollect_top<Src>(X, n, m, S, P.temperature, P.cand_theta, P.l2e_t, P.top_p, P.top_k, P.flags, sh, bank, row);
    cc = sh.cand_count;
    if (th >= 0.0f) {
      Pl.cand_theta = th;
      path |= kPathRecollect;
    } else {
      cc = (uint32_t)kCap + 1u;
    }
  }
  const bool ovf = cc > (uint32_t)kCap;
  const int c = ovf ? kCap : (int)cc;
  if (!ovf && c <= kShortMax && !(P.typical_p > 0.0f && P.typical_p < 1.0f)) {
    if (!select_short(Pl, Q, row, sh, c, m, S, path, u_row)) select_full_row<Src>(A, row, pen, sh, bank, m, S, path);
    return;
  }
  const int csort = next_pow2(c);
  for (int i = t; i < csort; i += kNT) {
    if (i < c) {
      const uint64_t a = sh.cand[i];
      const float p = __uint_as_float((uint32_t)(a >> 32)) / S;
      sh.cand[i] = ((uint64_t)(~__float_as_uint(p)) << 32) | (uint32_t)a;
    } else {
      sh.cand[i] = ~0ull;
    }
  }
  lds_barrier();
  lds_bitonic_sort_u64<kNT>(sh.cand, csort);

  // certified prefix: every element outside the list has p <= theta / S
  int M = 0;
  if (!ovf) {
    if (Pl.cand_theta <= 0.0f) {
      M = c;  // every element was collected
    } else {
      const float p_nc = Pl.cand_theta / S;
      uint32_t cnt = 0;
      for (int q = t; q < c; q += kNT) cnt += __uint_as_float(~(uint32_t)(sh.cand[q] >> 32)) > p_nc ? 1u : 0u;
      M = (int)wg_sum_sat<kNT>(cnt, 0x7fffffffu, sh.wg, bank);
    }
  }

  const LdsList LL{sh.cand};
  // a complete list bounds everything outside it: e < theta, p <= theta / S
  const float p_nc = ovf ? kInf : Pl.cand_theta / S;
  K = prefix_filters(LL, M, p_nc, n, P, S, sh, bank);
  const bool typical = P.typical_p > 0.0f && P.typical_p < 1.0f;
  const float u = u_row;
  bool fallback = K < 0;

  if (!fallback) {
    // ---- 5. typical-p on the kept prefix (:128-154)
    for (int q = t; q < kCap; q += kNT) sh.u.post.keep[q] = q < K ? 1 : 0;
    lds_barrier();
    if (typical && K == 1) {
      if (t == 0 && LL.p(0) > P.typical_p) sh.u.post.keep[0] = 0;
      lds_barrier();
    } else if (typical && K >= 2) {
      path |= kPathEntropy;
      {
        const EntropyResult er = entropy_pass<Src>(X, n, m, S, P.temperature, P.flags, sh, bank, row);
        H = er.H;
        bank = er.bank;
      }
      LLZ_STAMP(row, 12);
      const int ksort = next_pow2(K);
      for (int q = t; q < ksort; q += kNT) {
        if (q < K) {
          const float p = LL.p(q);
          const float surprise = p > 0.0f ? -log_f32(p) : kInf;
          const float dev = fabsf(surprise - H);
          sh.u.post.aux[q] = ((uint64_t)__float_as_uint(dev) << 32) | LL.id(q);
          sh.u.post.aux_pos[q] = (uint32_t)q;
        } else {
          sh.u.post.aux[q] = ~0ull;
          sh.u.post.aux_pos[q] = 0;
        }
      }
      lds_barrier();
      lds_bitonic_sort_kv<kNT>(sh.u.post.aux, sh.u.post.aux_pos, ksort);
      int st;
      seq_accumulate<false>(0.0f, K, P.typical_p, st, [&](int d) { return LL.p((int)sh.u.post.aux_pos[d]); },
                            sh, bank);
      if (st >= 0) {
        for (int d = st + t; d < K; d += kNT) sh.u.post.keep[sh.u.post.aux_pos[d]] = 0;
      }
      lds_barrier();
    }
    // ---- 6. total and draw (:156-168)
    total_and_draw(LL, K, [&](int q) { return sh.u.post.keep[q] != 0; }, u, total, token, consumed, sh, bank);

    // ---- outputs
    uint32_t kept = 0;
    for (int q = t; q < K; q += kNT) kept += sh.u.post.keep[q];
    kept = wg_sum_sat<kNT>(kept, 0x7fffffffu, sh.wg, bank);
    if (Q.kept_ids || Q.kept_probs) {
      // compact the kept positions in p order (thread-serial over K <= kCap)
      if (t == 0) {
        int o = 0;
        for (int q = 0; q < K && o < P.kept_cap; ++q) {
          if (sh.u.post.keep[q]) {
            if (Q.kept_ids) Q.kept_ids[(int64_t)row * P.kept_cap + o] = LL.id(q);
            if (Q.kept_probs) Q.kept_probs[(int64_t)row * P.kept_cap + o] = LL.p(q);
            ++o;
          }
        }
      }
    }
    if (t == 0) {
      Q.tokens[row] = token;
      if (Q.consumed) Q.consumed[row] = (uint8_t)consumed;
      if (Q.kept_count) Q.kept_count[row] = kept;
      if (Q.row_stats) {
        float* rs = Q.row_stats + (int64_t)row * 4;
        rs[0] = m; rs[1] = S; rs[2] = H; rs[3] = total;
      }
      if (Q.status) Q.status[row] = path;
    }
    return;
  }

  // ---- full-row fallback: every probability, stable radix sort, filters
  select_full_row<Src>(A, row, pen, sh, bank, m, S, path);
}

// The full-row fallback of k_select: every probability, stable radix sort of
// the whole row in the workspace, the filters and the draw over it.
// Typical-p over the full row (sampler.zig:128-154) in the full-row
// fallback.  What the reference's loop keeps is the selected elements before
// the first position of the typical order (dev ascending, index ascending
// among equal devs: std.mem.sort is stable) where the cumulative probability
// of the selected ones exceeds typical_p; so only the order's head up to that
// position is needed, not the whole row sorted by dev:
//  1. each element's dev key (the bits of dev >= 0; 0xffffffff when it is not
//     selected) in index order, and a histogram of the selected ones by the
//     key's top 11 bits (a monotone bucket of dev) with their count and an
//     approximate probability sum;
//  2. the head: the buckets up to the first one where the approximate
//     cumulative sum exceeds typical_p (1 + 2^-5);
//  3. the head's elements, in index order, sorted by key (stable);
//  4. the exact cumulative sum over the sorted head.  If it does not exceed
//     typical_p inside the head (the approximate sums misled, or the head is
//     everything), steps 1-4 run again with every selected element.
// Selected: the element's p-order position is below K, i.e. its key ~p bits
// pk and index i satisfy (pk, i) <= (keyK, idK), the key and id at position
// K - 1 (every element when K == n).  Returns the head's length C (sorted
// (key, id) in Ck, Cv), the first position st whose sum exceeds
// typical_p (-1: none, and then C == K), and the id of the row's first
// element in p order (p desc, id asc).
struct TypicalHead {
  int C, st;
  uint32_t first;
};

template <class Src>
__device__ TypicalHead typical_head(const Src& X, int n, float m, float S, float H, const RowParams& P, int K,
                                    uint32_t keyK, uint32_t idK, uint32_t* Bk, uint32_t* Bv, uint32_t* Ck,
                                    uint32_t* Cv, SampleShared& sh, int& bank) {
  constexpr int HB = 2048;  // histogram buckets: key >> 20 for keys <= 0x7fffffff
  constexpr int TV = 8;     // elements per thread per tile
  const int t = (int)threadIdx.x;
  const bool t1 = (P.flags & kFlagTIsOne) != 0;
  const bool vec = (P.flags & kFlagVecSrc) != 0;
  uint32_t* hcnt = sh.u.post.radix.stage_k;                        // [HB]
  float* hsum = reinterpret_cast<float*>(sh.u.post.radix.stage_v);  // [HB]
  TypicalHead r{0, -1, 0u};
  for (int attempt = 0; attempt < 2; ++attempt) {
    // ---- 1. dev keys (and on the first attempt the histogram)
    if (attempt == 0) {
      for (int b = t; b < HB; b += kNT) {
        hcnt[b] = 0u;
        hsum[b] = 0.0f;
      }
      lds_barrier();
    }
    uint32_t bpk = 0xffffffffu, bid = 0xffffffffu;  // this thread's first element in p order
    for (int base = 0; base < n; base += kNT * TV) {
      const int pos = base + t * TV;
      float va[kLaneV], vb[kLaneV];
      X.load4(pos, n, vec, va);
      X.load4(pos + kLaneV, n, vec, vb);
#pragma unroll
      for (int k = 0; k < TV; ++k) {
        const int i = pos + k;
        if (i < n) {
          const float p = row_exp(k < kLaneV ? va[k] : vb[k - kLaneV], m, P.temperature, t1) / S;
          const uint32_t pk = ~__float_as_uint(p);
          const bool sel = K >= n || pk < keyK || (pk == keyK && (uint32_t)i <= idK);
          const float surprise = p > 0.0f ? -log_f32(p) : kInf;
          const uint32_t dk = sel ? __float_as_uint(fabsf(surprise - H)) : 0xffffffffu;
          Bk[i] = dk;
          if (pk < bpk || (pk == bpk && (uint32_t)i < bid)) {
            bpk = pk;
            bid = (uint32_t)i;
          }
          if (attempt == 0 && sel) {
            atomicAdd(&hcnt[dk >> 20], 1u);
            atomicAdd(&hsum[dk >> 20], p);
          }
        }
      }
    }
    if (attempt == 0) {
      const uint32_t gpk = wg_min_u32<kNT>(bpk, sh.wg, bank);
      r.first = wg_min_u32<kNT>(bpk == gpk ? bid : 0xffffffffu, sh.wg, bank);
    }
    __threadfence();
    __syncthreads();
    // ---- 2. the head's last bucket (wave 0: 32 buckets per lane)
    if (wave_id() == 0) {
      int bstar = HB - 1;
      if (attempt == 0) {
        const int lane = lane_id();
        constexpr int PL = HB / kWave;
        float ls = 0.0f;
        for (int b = 0; b < PL; ++b) ls += hsum[lane * PL + b];
        const float incl = __uint_as_float(wave_incl_scan_op(__float_as_uint(ls), 0u, [](uint32_t a, uint32_t b) {
          return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
        }));
        const float thr = P.typical_p * (1.0f + 0x1p-5f);
        float run = incl - ls;
        int hit = HB;
        for (int b = 0; b < PL && hit == HB; ++b) {
          run += hsum[lane * PL + b];
          if (run > thr) hit = lane * PL + b;
        }
        const uint64_t hm = bal64(hit < HB);
        if (hm != 0ull) bstar = (int)readlane_u32((uint32_t)hit, __ffsll((long long)hm) - 1);
      }
      if (lane_id() == 0) sh.misc[2] = (uint32_t)bstar;
    }
    __syncthreads();
    const uint32_t bstar = sh.misc[2];
    // ---- 3. the head in index order
    int C = 0;
    for (int base = 0; base < n; base += kNT * TV) {
      const int pos = base + t * TV;
      uint32_t dk[TV];
      uint32_t cnt = 0;
#pragma unroll
      for (int k = 0; k < TV; ++k) {
        dk[k] = pos + k < n ? Bk[pos + k] : 0xffffffffu;
        cnt += (dk[k] != 0xffffffffu && (dk[k] >> 20) <= bstar) ? 1u : 0u;
      }
      uint32_t o = (uint32_t)C + wg_excl_scan_sat<kNT>(cnt, 0x7fffffffu, sh.wg, bank);
#pragma unroll
      for (int k = 0; k < TV; ++k) {
        if (dk[k] != 0xffffffffu && (dk[k] >> 20) <= bstar) {
          Ck[o] = dk[k];
          Cv[o] = (uint32_t)(pos + k);
          ++o;
        }
      }
      C += (int)wg_sum_sat<kNT>(cnt, 0x7fffffffu, sh.wg, bank);
    }
    __threadfence();
    __syncthreads();
    // ---- 4. sorted by key, then the exact cumulative sum
    wg_radix_sort_pairs<kNT>(Ck, Cv, Bk, Bv, C, sh.u.post.radix);
    __threadfence();
    __syncthreads();
    int st;
    list_accumulate<kNT, 2, false>(
        0.0f, C, P.typical_p, st,
        [&](int d) { return row_exp(X.at((int)Cv[d]), m, P.temperature, t1) / S; }, sh.wg, bank);
    r.C = C;
    r.st = st;
    if (st >= 0 || C >= K) break;
  }
  return r;
}

// Top-k / top-p / min-p, the total and the draw by buckets (llz_bucket.h)
// for a row without typical-p whose kept prefix overflowed the candidate
// list.  Ak: the row's key buffer (n words).  Returns false when the row
// needs the sorting path (nothing is written then but Ak).
template <class Src>
__device__ bool select_buckets(const Src& X, int n, float m, float S, float u, const RowParams& P, uint32_t* Ak,
                               SampleShared& sh, int& bank, BucketResult& res, int row) {
  BucketShared& bs = sh.u.bkt;
  const int t = (int)threadIdx.x;
  const bool t1 = (P.flags & kFlagTIsOne) != 0;
  const bool vec = (P.flags & kFlagVecSrc) != 0;
  const bool topp = P.top_p > 0.0f && P.top_p < 1.0f;
  if (n >= (1 << 20)) return false;  // histogram counts hold 20 bits
  const uint32_t Kk = (P.top_k > 0 && P.top_k < (uint32_t)n) ? P.top_k : (uint32_t)n;
  // probs[indices[0]] is the maximum's, whose e is exp(0) = 1 (sampler.zig:121)
  const float p0 = 1.0f / S;
  const float thr_m = p0 * P.min_p;
  const uint32_t kmin = ~__float_as_uint(p0);  // every key is at least this
  const double D = kBucketDelta;

  // ---- A: the exact p of every element (sampler.zig:85, :90), its key, and
  // the coarse histogram of a sample (every eighth element)
  // top binade of coarse bucket b (its smallest key); the last one holds every
  // key past the range too
  auto coarse_Etop = [&](int b) { return key_E(kmin + ((uint32_t)b << kCoarseShift)); };
  for (int b = t; b < kNB; b += kNT) bs.hist[bix(b)] = 0ull;
  lds_barrier();
  uint32_t km = 0, fk = 0xffffffffu, fid = 0xffffffffu;
  {
    constexpr int TV = RowTiles8::V;
    const RowTiles8 rt(X.x, n, vec);
    float raw[TV];
    rt.load(t * TV, raw);
    for (int base = 0; base < n; base += kNT * TV) {
      const int pos = base + t * TV;
      rt.fix_tail(pos, raw);
      float v[TV];
#pragma unroll
      for (int k = 0; k < TV; ++k) v[k] = pos + k < n ? X.fix(pos + k, raw[k]) : 0.0f;
      if (base + kNT * TV < n) rt.load(pos + kNT * TV, raw);
      uint32_t key[TV];
#pragma unroll
      for (int k = 0; k < TV; ++k) {
        const float p = row_exp(v[k], m, P.temperature, t1) / S;
        const bool in = pos + k < n;
        key[k] = in ? ~__float_as_uint(p) : 0xffffffffu;
        if (in) {
          km += p >= thr_m ? 1u : 0u;
          if (key[k] < fk) {  // positions ascend within a thread: the first of equal keys stays
            fk = key[k];
            fid = (uint32_t)(pos + k);
          }
          if (k == 0) {  // every eighth element, weight 8 (count and mass)
            const uint32_t cb = min((key[k] - kmin) >> kCoarseShift, (uint32_t)kNB - 1u);
            atomicAdd(&bs.hist[bix(cb)], 8ull * hist_word(key[k], coarse_Etop((int)cb)));
          }
        }
      }
      if (pos + TV <= n && (reinterpret_cast<uintptr_t>(Ak + pos) & 15u) == 0u) {
        *reinterpret_cast<uint4*>(Ak + pos) = make_uint4(key[0], key[1], key[2], key[3]);
        *reinterpret_cast<uint4*>(Ak + pos + 4) = make_uint4(key[4], key[5], key[6], key[7]);
      } else {
#pragma unroll
        for (int k = 0; k < TV; ++k)
          if (pos + k < n) Ak[pos + k] = key[k];
      }
    }
  }
  km = P.min_p > 0.0f ? wg_sum_sat<kNT>(km, 0x7fffffffu, sh.wg, bank) : (uint32_t)n;
  const uint32_t gk = wg_min_u32<kNT>(fk, sh.wg, bank);
  const uint32_t first = wg_min_u32<kNT>(fk == gk ? fid : 0xffffffffu, sh.wg, bank);  // indices[0]
  const uint32_t Lw = min(Kk, km);  // positions top-k and min-p keep
  __threadfence();
  __syncthreads();
  for (int b = t; b < kNB; b += kNT) hist_unpack(bs.hist[bix(b)], coarse_Etop(b), bs.cnt[bix(b)], bs.mass[bix(b)]);
  __syncthreads();
  LLZ_STAMP(row, 23);

  // ---- the region the chain can reach: coarse buckets up to the first whose
  // count reaches Lw or whose mass passes top-p, both with a margin for the
  // histogram's sampling (about sqrt(8 count): 0.6% at 217k elements); a cut
  // beyond the region only sends the row to the sorting path
  if (wave_id() == 0) {
    int cs = kNB - 1;
    bucket_scan(bs, [&](int b, uint32_t ec, double em) {
      const uint32_t ic = ec + bs.cnt[bix(b)];
      const double im = em + (double)bs.mass[bix(b)];
      if (b < cs && ((double)ic >= 1.05 * Lw + 2048.0 || (topp && im > (double)P.top_p * 1.05))) cs = b;
    });
    cs = (int)wave_min_u32((uint32_t)cs);
    if (lane_id() == 0) bs.ctl[0] = (uint32_t)cs;
  }
  __syncthreads();
  BucketRange br;
  {
    const uint64_t span = (uint64_t)(bs.ctl[0] + 1u) << kCoarseShift;
    int sh_f = 0;
    while ((span >> sh_f) > (uint64_t)kNB) ++sh_f;
    br.kmin = kmin;
    br.kcut = (uint32_t)min((uint64_t)kmin + span, (uint64_t)0xffffffffu);
    br.shift = sh_f;
  }
  // ---- A': the fine histogram of the region from the stored keys
  auto fine_Etop = [&](int b) { return key_E(br.kmin + ((uint32_t)b << br.shift)); };
  for (int b = t; b < kNB; b += kNT) bs.hist[bix(b)] = 0ull;
  lds_barrier();
  for (int base = 0; base < n; base += kNT * 8) {
    const int pos = base + t * 8;
    uint32_t k[8];
    bucket_keys8(Ak, pos, n, k);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (br.in(k[i])) {
        const int b = br.of(k[i]);
        atomicAdd(&bs.hist[bix(b)], hist_word(k[i], fine_Etop(b)));
      }
    }
  }
  __syncthreads();
  for (int b = t; b < kNB; b += kNT) hist_unpack(bs.hist[bix(b)], fine_Etop(b), bs.cnt[bix(b)], bs.mass[bix(b)]);
  __syncthreads();

  LLZ_STAMP(row, 24);
  // ---- the running sum of top-p and the total (sampler.zig:112-117, :156-159)
  if (wave_id() == 0) {
    bucket_scan(bs, [&](int b, uint32_t ec, double em) {
      const uint32_t c = bs.cnt[bix(b)];
      const uint32_t ic = ec + c;
      const double im = em + (double)bs.mass[bix(b)];
      uint8_t cl = kBExact;
      int j = 0;
      if (c == 0) {
        cl = kBEmpty;
      } else if (ec >= Lw || (topp && em * (1.0 - D) > (double)P.top_p)) {
        cl = kBNone;  // the chain stops before it
      } else {
        const double lo = em * (1.0 - D), hi = im * (1.0 + D);
        const int elo = dbl_binade(lo), ehi = dbl_binade(hi);
        const bool exact = b == 0 || (ec < Lw && Lw < ic) || (topp && hi > (double)P.top_p) || !(lo >= 0x1p-120) ||
                           elo != ehi || elo > 126;
        cl = exact ? kBExact : kBPlain;
        j = exact ? 0 : elo;
      }
      bs.cls[bix(b)] = cl;
      bs.jg[bix(b)] = (int8_t)j;
    });
  }
  __syncthreads();
  LLZ_STAMP(row, 25);
  float v, before;
  uint32_t pos, id;
  bool stop;
  uint32_t why = bucket_chain<false, kNT>(Ak, n, br, bs, 0.0f, Lw, topp ? P.top_p : -1.0f, v, before, pos, stop, id, row);
  if (why != 0u) {
    res.why = why;
    return false;
  }
  LLZ_STAMP(row, 26);
  const uint32_t K = pos;                  // the top-p cut, or Lw
  const float total = stop ? before : v;   // the sum of the kept prefix
  res.why = 0u;
  res.K = K;
  res.total = total;
  res.token = first;
  res.consumed = 0;
  if (!(total > 0.0f)) return true;  // sampler.zig:160: indices[0], no draw

  // ---- the draw (sampler.zig:162-168)
  const float r0 = u * total;
  if (wave_id() == 0) {
    bucket_scan(bs, [&](int b, uint32_t ec, double em) {
      const uint32_t c = bs.cnt[bix(b)];
      const uint32_t ic = ec + c;
      const double im = em + (double)bs.mass[bix(b)];
      uint8_t cl = kBExact;
      int j = 0;
      if (c == 0) {
        cl = kBEmpty;
      } else if (ec >= K || (double)r0 - em * (1.0 - D) <= 0.0) {
        cl = kBNone;  // past the kept prefix, or the draw stops before it
      } else {
        const double hi = (double)r0 - em * (1.0 - D);  // the value before the bucket, at most
        const double lo = (double)r0 - im * (1.0 + D);  // after it, at least
        const int elo = dbl_binade(lo), ehi = dbl_binade(hi);
        const bool exact = (ec < K && K < ic) || !(lo >= 0x1p-120) || elo != ehi || ehi > 126;
        cl = exact ? kBExact : kBPlain;
        j = exact ? 0 : elo;
      }
      bs.cls[bix(b)] = cl;
      bs.jg[bix(b)] = (int8_t)j;
    });
  }
  __syncthreads();
  LLZ_STAMP(row, 27);
  why = bucket_chain<true, kNT>(Ak, n, br, bs, r0, K, -1.0f, v, before, pos, stop, id, row);
  LLZ_STAMP(row, 28);
  if (why != 0u) {
    res.why = 32u + why;
    return false;
  }
  res.token = stop ? id : first;  // never at or below 0: indices[0]
  res.consumed = 1;
  return true;
}

template <class Src>
__device__ __noinline__ void select_full_row(const KArgs* A, int row, const PenShared* pen, SampleShared& sh,
                                             int bank, float m, float S, uint32_t path) {
  const RowParams& P = A->P;
  const RowPtrs& Q = A->Q;
  const Src X = make_src<Src>(P, Q, row, pen);
  const int t = (int)threadIdx.x;
  const int n = P.n;
  const bool t1 = (P.flags & kFlagTIsOne) != 0;
  const bool vec = (P.flags & kFlagVecSrc) != 0;
  const bool typical = P.typical_p > 0.0f && P.typical_p < 1.0f;
  const float u = Q.uniforms[row];
  int K = 0;
  float H = 0.0f, total = 0.0f;
  uint32_t token = 0, consumed = 0;
  path |= kPathFallback;
  if (!(P.flags & kFlagFallback)) {
    if (t == 0) {
      Q.tokens[row] = 0xffffffffu;
      if (Q.consumed) Q.consumed[row] = 0;
      if (Q.status) Q.status[row] = path | kPathError;
    }
    return;
  }
  // one of the call's fb_slots buffer sets, claimed for this row: a slot is
  // free for this call when its owner word holds anything but this call's
  // epoch.  At most fb_slots rows hold one at a time; a row that finds none
  // waits for a holder (a running workgroup that needs nothing else) to
  // release one.  The fences make the previous holder's writes, possibly
  // from another XCD's L2, land before this row touches the buffers.
  if (t == 0) {
    const unsigned long long E = P.epoch;
    int got = -1;
    for (uint32_t spin = 0; got < 0 && spin < (1u << 20); ++spin) {
      for (int k = 0; k < P.fb_slots && got < 0; ++k) {
        const int s = (row + k) % P.fb_slots;
        const unsigned long long old = __hip_atomic_load(&Q.fb_owner[s], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old != E && atomicCAS(&Q.fb_owner[s], old, E) == old) got = s;
      }
      if (got < 0) __builtin_amdgcn_s_sleep(127);
    }
    __threadfence();
    sh.misc[1] = (uint32_t)got;
  }
  __syncthreads();
  const int slot = (int)sh.misc[1];
  if (slot < 0 || slot >= P.fb_slots) {  // no slot within the wait bound
    if (t == 0) {
      Q.tokens[row] = 0xffffffffu;
      if (Q.consumed) Q.consumed[row] = 0;
      if (Q.status) Q.status[row] = path | kPathError;
    }
    return;
  }
  LLZ_STAMP(row, 8);
  const int64_t fo = (int64_t)slot * n;
  const int64_t fs = (int64_t)P.fb_slots * n;
  uint32_t* Ak = Q.fb + 0 * fs + fo;
  uint32_t* Av = Q.fb + 1 * fs + fo;
  uint32_t* Bk = Q.fb + 2 * fs + fo;
  uint32_t* Bv = Q.fb + 3 * fs + fo;
  uint32_t* Ck = Q.fb + 4 * fs + fo;
  uint32_t* Cv = Q.fb + 5 * fs + fo;
  uint8_t* mask = Q.fb_mask + fo;
  // With typical-p and no prefix filter every element is selected (K = n),
  // and the p order matters only among the elements typical-p keeps: the
  // whole row is then never sorted by p.
  const bool filters = (P.top_k > 0 && P.top_k < (uint32_t)n) || (P.top_p > 0.0f && P.top_p < 1.0f) ||
                       P.min_p > 0.0f;
  const bool lazy_p = typical && !filters && n >= 2;
  // release the slot once every thread is done with it (a value no later
  // call's epoch takes)
  auto release = [&]() {
    __threadfence();
    __syncthreads();
    LLZ_STAMP(row, 14);
    if (t == 0) atomicExch(&Q.fb_owner[slot], P.epoch ^ (1ull << 63));
  };
  // Without typical-p the kept prefix, the total and the draw come from
  // buckets of the p keys (llz_bucket.h), without a sort of the row.  The
  // kept ids in p order (a diagnostic output) need the sort.
  if (!typical && filters && !Q.kept_ids && !Q.kept_probs && n >= kBucketMinN) {
    BucketResult br;
    br.why = 0u;
    if (select_buckets<Src>(X, n, m, S, u, P, Ak, sh, bank, br, row)) {
      LLZ_STAMP(row, 11);
      if (t == 0) {
        Q.tokens[row] = br.token;
        if (Q.consumed) Q.consumed[row] = (uint8_t)br.consumed;
        if (Q.kept_count) Q.kept_count[row] = br.K;
        if (Q.row_stats) {
          float* rs = Q.row_stats + (int64_t)row * 4;
          rs[0] = m; rs[1] = S; rs[2] = 0.0f; rs[3] = br.total;
        }
        if (Q.status) Q.status[row] = path | kPathBuckets;
      }
      release();
      return;
    }
    __syncthreads();  // every thread is past the bucket path: the sort below overwrites its keys
    path |= min(br.why, 255u) << 8;  // diagnostic: why the bucket path declined
  }
  const GlobalList GL{Ak, Av};
  if (!lazy_p) {
    // (~p bits, id) in index order, the next tile's loads in flight; the
    // smallest key lets the sort skip the digits every key shares
    constexpr int TV = RowTiles8::V;
    const RowTiles8 rt(X.x, n, vec);
    float raw[TV];
    rt.load(t * TV, raw);
    uint32_t kmin = 0xffffffffu;
    for (int base = 0; base < n; base += kNT * TV) {
      const int pos = base + t * TV;
      rt.fix_tail(pos, raw);  // also in the first tile: a span crossing the row's end
      float v[TV];
#pragma unroll
      for (int k = 0; k < TV; ++k) v[k] = pos + k < n ? X.fix(pos + k, raw[k]) : 0.0f;
      if (base + kNT * TV < n) rt.load(pos + kNT * TV, raw);
#pragma unroll
      for (int k = 0; k < TV; ++k) {
        if (pos + k < n) {
          const uint32_t key = ~__float_as_uint(row_exp(v[k], m, P.temperature, t1) / S);
          kmin = min(kmin, key);
          Ak[pos + k] = key;
          Av[pos + k] = (uint32_t)(pos + k);
        }
      }
    }
    kmin = wg_min_u32<kNT>(kmin, sh.wg, bank);
    __threadfence();
    __syncthreads();
    LLZ_STAMP(row, 9);
    wg_radix_sort_pairs<kNT>(Ak, Av, Bk, Bv, n, sh.u.post.radix, kmin);
    __threadfence();
    __syncthreads();
    LLZ_STAMP(row, 10);
    K = prefix_filters(GL, n, kInf, n, P, S, sh, bank);  // M = n: never -1
    LLZ_STAMP(row, 11);
    if (K < 0) K = 0;
  } else {
    K = n;
  }

  // The final list (the kept elements among positions [0, Kf) of a list in
  // p order) and its outputs.
  auto finish = [&](const auto& L, int Kf, auto keep, uint32_t first) {
    total_and_draw(L, Kf, keep, u, total, token, consumed, sh, bank, first);
    uint32_t kept = 0;
    for (int q = t; q < Kf; q += kNT) kept += keep(q) ? 1u : 0u;
    kept = wg_sum_sat<kNT>(kept, 0x7fffffffu, sh.wg, bank);
    if (t == 0) {
      if (Q.kept_ids || Q.kept_probs) {  // thread-serial: diagnostic use only
        int o = 0;
        for (int q = 0; q < Kf && o < P.kept_cap; ++q) {
          if (keep(q)) {
            if (Q.kept_ids) Q.kept_ids[(int64_t)row * P.kept_cap + o] = L.id(q);
            if (Q.kept_probs) Q.kept_probs[(int64_t)row * P.kept_cap + o] = L.p(q);
            ++o;
          }
        }
      }
      Q.tokens[row] = token;
      if (Q.consumed) Q.consumed[row] = (uint8_t)consumed;
      if (Q.kept_count) Q.kept_count[row] = kept;
      if (Q.row_stats) {
        float* rs = Q.row_stats + (int64_t)row * 4;
        rs[0] = m; rs[1] = S; rs[2] = H; rs[3] = total;
      }
      if (Q.status) Q.status[row] = path;
    }
  };

  if (typical && K >= 2) {
    path |= kPathEntropy;
    {
      const EntropyResult er = entropy_pass<Src>(X, n, m, S, P.temperature, P.flags, sh, bank, row);
      H = er.H;
      bank = er.bank;
    }
    LLZ_STAMP(row, 12);
    const uint32_t keyK = K < n ? Ak[K - 1] : 0u;
    const uint32_t idK = K < n ? Av[K - 1] : 0u;
    const TypicalHead th = typical_head<Src>(X, n, m, S, H, P, K, keyK, idK, Bk, Bv, Ck, Cv, sh, bank);
    LLZ_STAMP(row, 13);
    // the cut: the first element of the typical order that is not kept
    const bool cut = th.st >= 0;
    const uint32_t dkc = cut ? Ck[th.st] : 0u, idc = cut ? Cv[th.st] : 0u;
    if (!lazy_p) {
      // keep flags in p order: (dev key, id) before the cut's
      for (int q = t; q < K; q += kNT) {
        const float p = GL.p(q);
        const float surprise = p > 0.0f ? -log_f32(p) : kInf;
        const uint32_t dk = __float_as_uint(fabsf(surprise - H));
        const uint32_t id = GL.id(q);
        mask[q] = (!cut || dk < dkc || (dk == dkc && id < idc)) ? 1 : 0;
      }
      __threadfence();
      __syncthreads();
      finish(GL, K, [&](int q) { return mask[q] != 0; }, 0xffffffffu);
    } else {
      // the kept elements are the head's first keep_n; put them in p order
      const int keep_n = cut ? th.st : th.C;
      if (keep_n <= kCap) {
        const int ks = next_pow2(max(keep_n, 1));
        for (int d = t; d < ks; d += kNT) {
          if (d < keep_n) {
            const uint32_t id = Cv[d];
            const float p = row_exp(X.at((int)id), m, P.temperature, t1) / S;
            sh.cand[d] = ((uint64_t)(~__float_as_uint(p)) << 32) | id;
          } else {
            sh.cand[d] = ~0ull;
          }
        }
        lds_barrier();
        lds_bitonic_sort_u64<kNT>(sh.cand, ks);
        lds_barrier();
        finish(LdsList{sh.cand}, keep_n, [&](int) { return true; }, th.first);
      } else {
        // by id, then stably by ~p bits: (p desc, id asc)
        for (int d = t; d < keep_n; d += kNT) {
          const uint32_t id = Cv[d];
          const float p = row_exp(X.at((int)id), m, P.temperature, t1) / S;
          Ak[d] = id;
          Av[d] = ~__float_as_uint(p);
        }
        __threadfence();
        __syncthreads();
        wg_radix_sort_pairs<kNT>(Ak, Av, Bk, Bv, keep_n, sh.u.post.radix);
        __threadfence();
        __syncthreads();
        wg_radix_sort_pairs<kNT>(Av, Ak, Bk, Bv, keep_n, sh.u.post.radix);
        __threadfence();
        __syncthreads();
        finish(GlobalList{Av, Ak}, keep_n, [&](int) { return true; }, th.first);
      }
    }
  } else if (typical && K == 1) {
    const bool k0 = !(GL.p(0) > P.typical_p);
    finish(GL, K, [&](int) { return k0; }, 0xffffffffu);
  } else {
    finish(GL, K, [&](int) { return true; }, 0xffffffffu);
  }
  release();
}

}  // namespace llz
