// llz_stats.hip -- k_stats: the fused per-row sampling kernel.  Phases L .. C
// compute the row statistics (sampler.zig:80-88): the row maximum, the exact
// sequential f32 normaliser and the candidate list, with one HBM read per
// logit (method and error bound in llz_fast.h).  The same workgroup then runs
// the selection stage (llz_select.h, sampler.zig:89-168); a row the fast path
// cannot certify takes the streaming normaliser there instead.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "llz_exact.h"
#include "llz_fast.h"
#include "llz_internal.h"
#include "llz_math.h"
#include "llz_norm.h"
#include "llz_select.h"
#include "llz_split.h"
#include "llz_token.h"
#include "llz_wg.h"

namespace llz {
namespace {

using namespace fastp;
constexpr float kInfS = __builtin_inff();
constexpr int kScanDepth = 8;  // rows beyond the single pass: float4 loads in flight per thread in the max scan



__device__ __forceinline__ float wave_incl_scan_f32(float v) {
  return __uint_as_float(wave_incl_scan_op(__float_as_uint(v), 0u, [](uint32_t a, uint32_t b) {
    return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
  }));
}

__device__ __forceinline__ llz_f4v to_v4(float4 f) {
  llz_f4v v;
  v.x = f.x;
  v.y = f.y;
  v.z = f.z;
  v.w = f.w;
  return v;
}

__device__ __forceinline__ float4 neg_inf4() { return make_float4(-kInfS, -kInfS, -kInfS, -kInfS); }

// Branch-free segment loads (no per-lane branch, so every load of a wave can
// be in flight at once).  Absent positions read a valid address and are
// replaced by -inf.  ld4: 16-byte aligned row with n % 4 == 0.
__device__ __forceinline__ float4 ld4(const float* xr, int pos, int n) {
  const bool in = pos < n;
  const float4 v = ld_nt4(xr + (in ? pos : 0));
  return in ? v : neg_inf4();
}
__device__ __forceinline__ float4 ld1x4(const float* xr, int pos, int n) {
  float4 v;
  v.x = xr[pos + 0 < n ? pos + 0 : 0];
  v.y = xr[pos + 1 < n ? pos + 1 : 0];
  v.z = xr[pos + 2 < n ? pos + 2 : 0];
  v.w = xr[pos + 3 < n ? pos + 3 : 0];
  if (pos + 0 >= n) v.x = -kInfS;
  if (pos + 1 >= n) v.y = -kInfS;
  if (pos + 2 >= n) v.z = -kInfS;
  if (pos + 3 >= n) v.w = -kInfS;
  return v;
}

// Copy one segment (1 KB) of the row into an LDS block of 256 floats:
// straight to LDS when the segment is full and aligned, else through VGPRs.
__device__ __forceinline__ void seg_to_lds(const float* xr, int seg, int n, bool fastld, float* dst) {
  const int lane = lane_id();
  const int pos = seg * SEG + lane * 4;
  if (fastld && (seg + 1) * SEG <= n) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_global_load_lds(xr + pos, dst, 16, 0, 0);
#endif
  } else {
    *reinterpret_cast<float4*>(dst + lane * 4) = fastld ? ld4(xr, pos, n) : ld1x4(xr, pos, n);
  }
}

__device__ __forceinline__ float4 q_of(float4 v, float l2e_t, float cw) {
  float4 q;
  q.x = __builtin_amdgcn_exp2f(fmaf(v.x, l2e_t, -cw));
  q.y = __builtin_amdgcn_exp2f(fmaf(v.y, l2e_t, -cw));
  q.z = __builtin_amdgcn_exp2f(fmaf(v.z, l2e_t, -cw));
  q.w = __builtin_amdgcn_exp2f(fmaf(v.w, l2e_t, -cw));
  return q;
}

__device__ __forceinline__ float max4(float4 v) { return fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)); }

__device__ __forceinline__ void push_cand(FastShared& F, const RowPtrs& Q, int row, float e, uint32_t id) {
  const uint32_t slot = atomicAdd(&F.ncand, 1u);
  if (slot < (uint32_t)kCandCap) Q.cand[(int64_t)row * kCandCap + slot] = ((uint64_t)__float_as_uint(e) << 32) | id;
}

// EXACT slots per wave: slot 0 on wave 0 alone, slots 1.. on waves 1 .. W-1
// in turn (slot s on wave 1 + (s - 1) % (W - 1)).  Slot 0 is the row's first
// segment in the first round, which wave 0 then sums term by term; the other
// waves take the slots that need tables.  Wave w's slots: w, w + slot_step(w), ...
__device__ __forceinline__ int slot_step(int w) { return w == 0 ? DCAP : W - 1; }

// Issue the re-reads of this wave's EXACT slots into their dump areas (the
// caller waits for them).
template <bool FASTLD>
__device__ __forceinline__ void exact_loads(FastShared& F, const float* xr, int w, int nslot, int n) {
  for (int slot = w; slot < nslot; slot += slot_step(w)) seg_to_lds(xr, F.slotseg[slot], n, FASTLD, &F.u.x.dump[slot][0]);
}

// The exact terms of four consecutive positions (sampler.zig:85), without
// branches per term.
__device__ __forceinline__ float4 exact_terms4(float4 v, float m, float T, bool t1) {
  float x0 = v.x - m, x1 = v.y - m, x2 = v.z - m, x3 = v.w - m;
  if (!t1) {
    x0 = x0 / T;
    x1 = x1 / T;
    x2 = x2 / T;
    x3 = x3 / T;
  }
  return make_float4(exp_f32(x0), exp_f32(x1), exp_f32(x2), exp_f32(x3));
}

// The exact terms of EXACT slot `slot` (loaded and waited for) into its dump
// area, and its candidates (once per segment).
template <class Src>
__device__ __forceinline__ void slot_terms(FastShared& F, const RowPtrs& Q, const RowParams& P, const Src& X,
                                           int row, int slot, int n, float m, float theta, bool t1) {
  const int lane = lane_id();
  const int seg = F.slotseg[slot];
  const bool pred = F.sflag[seg] == EXACT_PRED;
  float4* p = reinterpret_cast<float4*>(&F.u.x.dump[slot][lane * 4]);
  const int pos = seg * SEG + lane * 4;
  float4 e = exact_terms4(X.fix4(pos, *p, n), m, P.temperature, t1);
  e.x = pos + 0 < n ? e.x : 0.0f;
  e.y = pos + 1 < n ? e.y : 0.0f;
  e.z = pos + 2 < n ? e.z : 0.0f;
  e.w = pos + 3 < n ? e.w : 0.0f;
  *p = e;
  // candidates (absent positions hold 0 < theta)
  const bool cand_any = e.x >= theta || e.y >= theta || e.z >= theta || e.w >= theta;
  if (bal64(pred && cand_any) != 0ull) {
    const float es[4] = {e.x, e.y, e.z, e.w};
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (pred && es[c] >= theta) push_cand(F, Q, row, es[c], (uint32_t)(pos + c));
  }
  if (pred && lane == 0) F.sflag[seg] = EXACT_DONE;  // a later round must not collect them again
}

// The per-lane inclusive prefix tables of slot `slot`'s exact terms rounded
// on grids sj .. sj + sng - 1, with the lanes holding a tie: grids J0 and
// J0 + 1 (the common case: a segment crossing one binade boundary) in one
// pass, further grids one at a time.
__device__ __forceinline__ void slot_tables(FastShared& F, int slot) {
  const int lane = lane_id();
  const int seg = F.slotseg[slot];
  const float4 e = *reinterpret_cast<const float4*>(&F.u.x.dump[slot][lane * 4]);
  const float es[4] = {e.x, e.y, e.z, e.w};
  const int J0 = F.sj[seg];
  const int ng = F.sng[seg];
  {
    uint32_t sa = 0, sb = 0;
    bool ta = false, tb = false;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      bool tie;
      sa = sat_add(sa, grid_round(es[c], J0, tie), kSat);
      ta = ta || tie;
      sb = sat_add(sb, grid_round(es[c], J0 + 1, tie), kSat);
      tb = tb || tie;
    }
    const uint32_t pa = wave_incl_scan_sat(sa, kSat);
    const uint32_t pb = wave_incl_scan_sat(sb, kSat);
    const uint64_t ma = bal64(ta), mb = bal64(tb);
    F.u.x.pref[slot][0][lane] = pa;
    F.u.x.pref[slot][1][lane] = pb;  // NG >= 2: room even when ng == 1
    if (lane == 0) {
      F.u.x.tmask[slot][0] = ma;
      F.u.x.tmask[slot][1] = mb;
    }
  }
  for (int kk = 2; kk < ng; ++kk) {
    uint32_t sum = 0;
    bool tie_any = false;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      bool tie;
      sum = sat_add(sum, grid_round(es[c], J0 + kk, tie), kSat);
      tie_any = tie_any || tie;
    }
    F.u.x.pref[slot][kk][lane] = wave_incl_scan_sat(sum, kSat);
    const uint64_t tm = bal64(tie_any);
    if (lane == 0) F.u.x.tmask[slot][kk] = tm;
  }
}

// Rounds after the first: the terms and tables of this wave's slots (slot s
// on its wave (slot_step), all loaded by this wave and waited for).
template <class Src>
__device__ __forceinline__ void exact_segments(FastShared& F, const RowPtrs& Q, const RowParams& P, const Src& X,
                                               int row, int w, int nslot, int n, float m, float theta, bool t1) {
  for (int slot = w; slot < nslot; slot += slot_step(w)) {
    slot_terms(F, Q, P, X, row, slot, n, m, theta, t1);
    slot_tables(F, slot);
  }
}

// Combine wave: the exact accumulation of lanes p.. of a segment's exact
// terms (x) from s by the generic exact method (llz_norm.h), for a running
// sum outside the tabulated grids: a segment holding a term far above the
// running sum, or a prediction miss.  Out of line: it is rare.
__device__ __noinline__ float resolve_generic(float s, float x0, float x1, float x2, float x3, int p) {
  const int lane = lane_id();
  const bool live = lane >= p;
  const float x[4] = {live ? x0 : -0.0f, live ? x1 : -0.0f, live ? x2 : -0.0f, live ? x3 : -0.0f};
  return wave_accumulate<4>(s, x);
}

// Wave-uniform copies (scalar registers): values every lane read from the
// same LDS address, or computed from such values, are uniform, but the
// compiler cannot prove it and would otherwise branch on them lane by lane.
__device__ __forceinline__ float uni_f(float x) { return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x))); }
__device__ __forceinline__ uint32_t uni_u(uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)x); }
__device__ __forceinline__ uint64_t uni_u64(uint64_t x) {
  return ((uint64_t)uni_u((uint32_t)(x >> 32)) << 32) | uni_u((uint32_t)x);
}

// An EXACT slot's data as the walk needs it, read ahead of its entry (it does
// not depend on the running sum): the lane's four exact terms and the prefix
// tables and tie masks of the slot's first two grids (loads in flight until
// first use).
struct SlotAhead {
  float4 e4;
  uint32_t pv0, pv1;
  uint32_t tm0l, tm0h, tm1l, tm1h;
};

__device__ __forceinline__ SlotAhead slot_ahead(const FastShared& F, int slot) {
  const int lane = lane_id();
  SlotAhead X;
  X.e4 = *reinterpret_cast<const float4*>(&F.u.x.dump[slot][lane * 4]);
  X.pv0 = F.u.x.pref[slot][0][lane];
  X.pv1 = F.u.x.pref[slot][1][lane];
  const uint64_t t0 = F.u.x.tmask[slot][0], t1 = F.u.x.tmask[slot][1];
  X.tm0l = (uint32_t)t0;
  X.tm0h = (uint32_t)(t0 >> 32);
  X.tm1l = (uint32_t)t1;
  X.tm1h = (uint32_t)(t1 >> 32);
  return X;
}

// Combine wave: the exact sequential sum across EXACT segment `slot`, using
// its prefix tables (grids J0 .. J0 + ng - 1) between events and replaying
// the lane that holds an event term by term.  The running sum is N on grid j
// (N * 2^(j-23), N < 2^24), kept in scalar registers; the slot's data was
// read ahead into X.
__device__ __forceinline__ void resolve_ahead(uint32_t& N_io, int& j_io, int slot, int J0, int ng,
                                              const SlotAhead& X, FastShared& F) {
  const int lane = lane_id();
  uint32_t N = N_io;
  int j = j_io;
  int p = 0;  // first lane not consumed
  if (j == J0 + 1 && ng >= 2) {
    // the sum crossed into the segment's second grid before it (a segment
    // with no event there adds the table's total)
    const uint32_t T1 = readlane_u32(X.pv1, kWave - 1);
    const uint64_t tm1 = ((uint64_t)uni_u(X.tm1h) << 32) | uni_u(X.tm1l);
    if (tm1 == 0ull && T1 < kSat && N + T1 < kGridTop) {
      N_io = N + T1;
      return;
    }
  }
  if (j == J0) {
    // the common case, short on dependent steps (a wave running alone waits
    // out each one): every lane replays its own four terms from the table's
    // prefix before it, as if it held the first event, while the event lane
    // is found; then at most one crossing into grid J0 + 1, where the rest of
    // the segment is one table difference
    const uint32_t before = N + wave_shift_up1(X.pv0);  // lane 0: N
    float t = __uint_as_float(grid_bits(before, j));
    t = t + X.e4.x;
    t = t + X.e4.y;
    t = t + X.e4.z;
    t = t + X.e4.w;
    const uint64_t tm0 = ((uint64_t)uni_u(X.tm0h) << 32) | uni_u(X.tm0l);
    const uint64_t ev = bal64(X.pv0 >= kSat || N + X.pv0 >= kGridTop) | tm0;
    // three outcomes, computed together and taken with one branch: no event
    // on grid J0 (the table's total), an event in the last lane, or one
    // crossing into grid J0 + 1 with the rest of the segment event-free there
    const int E = ev != 0ull ? __ffsll((long long)ev) - 1 : kWave - 1;
    const Grid g = grid_of(uni_f(readlane_f32(t, E)));
    const uint32_t T0 = readlane_u32(X.pv0, kWave - 1);
    const uint32_t B = readlane_u32(X.pv1, E), T = readlane_u32(X.pv1, kWave - 1);
    const uint64_t tm1 = ((uint64_t)uni_u(X.tm1h) << 32) | uni_u(X.tm1l);
    const uint64_t live1 = E < kWave - 1 ? (~0ull << (E + 1)) : 0ull;
    const bool none = ev == 0ull;
    const bool last = !none && E == kWave - 1;
    // table entries are saturating prefix sums: T - B is exact below kSat
    const bool cross = !none && !last && g.j == J0 + 1 && ng >= 2 && T < kSat && g.N + (T - B) < kGridTop &&
                       (tm1 & live1) == 0ull;
    if (none || last || cross) {
      N_io = none ? N + T0 : (last ? g.N : g.N + (T - B));
      j_io = none ? j : g.j;
      return;
    }
    // anything else: the general steps below, from the first event on
    N = g.N;
    j = g.j;
    p = E + 1;
  }
  // selects rather than branches: a taken branch costs a wave running alone
  // far more than the few operations it would skip
  for (int guard = 0; guard <= kWave && p < kWave; ++guard) {
    const int k = j - J0;
    uint32_t pv;
    uint64_t tm;
    if ((uint32_t)k < 2u && k < ng) {
      const uint32_t pv0 = X.pv0, pv1 = X.pv1;
      pv = k == 0 ? pv0 : pv1;
      asm volatile("" : "+v"(pv));
      tm = ((uint64_t)uni_u(k == 0 ? X.tm0h : X.tm1h) << 32) | uni_u(k == 0 ? X.tm0l : X.tm1l);
    } else if (k >= 2 && k < ng) {
      pv = F.u.x.pref[slot][k][lane];
      asm volatile("" : "+v"(pv));
      tm = uni_u64(F.u.x.tmask[slot][k]);
    } else {
      const float s = uni_f(resolve_generic(__uint_as_float(grid_bits(N, j)), X.e4.x, X.e4.y, X.e4.z, X.e4.w, p));
      if (lane == 0) F.diag |= kPathResolveGeneric;
      const Grid g = grid_of(s);
      N = g.N;
      j = g.j;
      break;
    }
    const uint32_t base_l = readlane_u32(pv, (p - 1) & (kWave - 1));
    const uint32_t base = p > 0 ? base_l : 0u;
    const uint64_t live = ~0ull << p;
    const bool cr = lane >= p && (pv >= kSat || N + (pv - base) >= kGridTop);
    // every lane from p replays its own four terms (sampler.zig:87) from the
    // table's integer before it, as if it held the first event: one readlane
    // of the event lane's result instead of four dependent steps
    const uint32_t before = N + (wave_shift_up1(pv) - base);  // lane p: N
    float t = __uint_as_float(grid_bits(before, j));
    t = t + X.e4.x;
    t = t + X.e4.y;
    t = t + X.e4.z;
    t = t + X.e4.w;
    const uint64_t ev = (bal64(cr) | tm) & live;
    if (ev == 0ull) {
      N = uni_u(N + (readlane_u32(pv, kWave - 1) - base));
      break;
    }
    const int E = __ffsll((long long)ev) - 1;
    const Grid g = grid_of(uni_f(readlane_f32(t, E)));
    N = g.N;
    j = g.j;
    p = E + 1;
  }
  N_io = N;
  j_io = j;
}

// Owner wave: settle its queued lanes (v4q[h]: the re-read logits of entry
// h * 64 + lane, four consecutive positions from the entry's position).
// Each term's lower-bracket rounding is recomputed exactly as phase S summed
// it; the terms it could not certify are evaluated with the exact exp and
// the difference corrects the segment sum.  Candidates are collected, and
// per segment with ties the units they add (PLAIN_TIE, sbump).  A
// segment's lanes are always queued and settled together, so the parity of
// the integer sum before a tie (all that decides it) is that of the lane's
// queued prefix, plus the corrections of the segment's lanes below it, plus
// the lane's exact roundings before it.
// v4q: the queued lanes' logits as the chain reads them, or raw (kXmCap:
// phase L's estimate and the exact value are both taken from them here).
template <int XM, class Src>
__device__ __forceinline__ void settle_specials(FastShared& F, const RowPtrs& Q, const RowParams& P, const Src& X,
                                                int row, int w, int qn, const float4 (&v4q)[2], float Rw, float cw,
                                                float m, float theta, bool t1) {
  const int lane = lane_id();
  const float bw = F.bw[w];  // |aw| of this wave (phase M)
  const int n = P.n;
  uint32_t pos2[2] = {0u, 0u}, pre2[2] = {0u, 0u}, rl[2][4] = {}, rx[2][4] = {};
  int j2[2] = {0, 0};
  bool act2[2] = {false, false};
  uint32_t spm = 0;
  // brackets as phase S computed them (the second half only when in use)
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (h == 1 && qn <= kWave) break;
    const int i = h * kWave + lane;
    act2[h] = i < qn;
    const uint32_t qp = act2[h] ? F.qpos[w][i] : 0u;
    pos2[h] = qp & 0x7fffffffu;
    pre2[h] = qp >> 31;  // parity: only that decides a tie
    j2[h] = F.sj[pos2[h] >> 8];
    const GridConst gc = grid_const(j2[h], Rw, theta, bw, t1, P.est_xe);
    const uint32_t tspec = __float_as_uint(gc.tspec);
    const float vv[4] = {v4q[h].x, v4q[h].y, v4q[h].z, v4q[h].w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bool present = act2[h] && (int)pos2[h] + c < n;
      float vq = vv[c];
      if constexpr (XM == kXmCap) {  // phase L's estimate of the soft-capped (and penalised) logit
        vq = cap_est(vq, P.cap_a2, P.cap_c);
        if (present && (X.xf & kXfPen) && X.penalised((int)pos2[h] + c)) vq = pen_est(vq, P.rpen, P.rpen_inv);
      }
      const float q = present ? __builtin_amdgcn_exp2f(fmaf(vq, P.l2e_t, -cw)) : 0.0f;  // phase L's q, bit for bit
      const uint32_t lo = __float_as_uint(fmaf(q, gc.sc_lo, MAGIC));
      const uint32_t hi = __float_as_uint(fmaf(q, gc.sc_hi, MAGIC));
      rl[h][c] = lo - MAGIC_BITS;
      rx[h][c] = rl[h][c];
      if (present && (lo != hi || hi >= tspec)) spm |= 1u << (4 * h + c);
    }
  }
  // exact roundings of the special terms (about one per lane)
  uint32_t tiem = 0, rem = spm;
  while (rem != 0u) {
    const int bt = __ffs(rem) - 1;
    rem &= rem - 1u;
    const int h = bt >> 2, c = bt & 3;
    const float4 vh = h == 0 ? v4q[0] : v4q[1];
    float v = c == 0 ? vh.x : c == 1 ? vh.y : c == 2 ? vh.z : vh.w;
    if constexpr (XM == kXmCap) v = X.fix((int)(h == 0 ? pos2[0] : pos2[1]) + c, v);  // the exact value
    const float e = exact_term(v, m, P.temperature, t1);
    bool tie;
    const uint32_t r = grid_round(e, h == 0 ? j2[0] : j2[1], tie);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) rx[hh][cc] = bt == 4 * hh + cc ? r : rx[hh][cc];
    if (tie) tiem |= 1u << bt;
    if (e >= theta) push_cand(F, Q, row, e, (h == 0 ? pos2[0] : pos2[1]) + (uint32_t)c);
  }
  uint32_t corr2[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    corr2[h] = (rx[h][0] - rl[h][0]) + (rx[h][1] - rl[h][1]) + (rx[h][2] - rl[h][2]) + (rx[h][3] - rl[h][3]);
    if (act2[h] && corr2[h] != 0u) atomicAdd(&F.v.ssum4[pos2[h] >> 8][0], corr2[h]);
  }
  if (bal64(tiem != 0u) == 0ull) return;

  // ties (rare): the integer sum before each, then per segment the units
  // its ties add for an even and an odd starting integer (a tie rounds up
  // when the running integer before it plus its rounding down is odd; the
  // running integer's parity depends on the start only through its parity)
  uint32_t tpos = 0xffffffffu, tpre = 0, tk = 0;  // this wave's ties, one per lane
  int nt = 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint64_t lanes = bal64((tiem >> (4 * h)) & 15u);
    while (lanes != 0ull) {
      const int L = __ffsll((long long)lanes) - 1;
      lanes &= lanes - 1ull;
      const uint32_t p4 = readlane_u32(pos2[h], L);
      // corrections of the segment's lanes below this one
      uint32_t c = 0;
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
        if (act2[h2] && (pos2[h2] >> 8) == (p4 >> 8) && pos2[h2] < p4) c += corr2[h2];
      const uint32_t below = readlane_u32(pre2[h], L) + wave_sum_u32(c);
      const uint32_t tb = readlane_u32((tiem >> (4 * h)) & 15u, L);
      uint32_t within = 0;
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        const uint32_t r = readlane_u32(rx[h][cc], L);
        if ((tb >> cc) & 1u) {
          if (lane == nt) {
            tpos = p4 + (uint32_t)cc;
            tpre = below + within;
            tk = r;
          }
          ++nt;
        }
        within += r;
      }
      if (nt > kWave - 4) break;
    }
  }
  if (nt > kWave - 4) {
    if (lane == 0) atomicOr(&F.fail, 1u);
    return;
  }
  bool open_t = lane < nt;
  while (bal64(open_t) != 0ull) {
    // the segment of the first remaining tie, its ties in position order
    const uint32_t g = wave_min_u32(open_t ? tpos : 0xffffffffu) >> 8;
    bool mine = open_t && (tpos >> 8) == g;
    uint32_t b0 = 0, b1 = 0;
    while (bal64(mine) != 0ull) {
      const uint32_t pmin = wave_min_u32(mine ? tpos : 0xffffffffu);
      const int L = __ffsll((long long)bal64(mine && tpos == pmin)) - 1;
      const uint32_t pr = readlane_u32(tpre, L), kk = readlane_u32(tk, L);
      b0 += ((0u + pr + b0 + kk) & 1u);
      b1 += ((1u + pr + b1 + kk) & 1u);
      mine = mine && tpos != pmin;
    }
    if (lane == 0) {
      if (b0 > 15u || b1 > 15u) atomicOr(&F.fail, 1u);
      F.sbump[g] = (uint8_t)(min(b0, 15u) | (min(b1, 15u) << 4));
      F.sflag[g] = PLAIN_TIE;
    }
    open_t = open_t && (tpos >> 8) != g;
  }
}

// Shared memory of k_stats.
union StatsShared {
  FastShared fast;      // phases L .. C
  SampleShared select;  // then the selection stage
};

// The next row beyond the grid for a workgroup that finished one: a counter
// word tagged with the low 40 bits of the call's epoch (a word left by
// another call, or not yet written, counts as 0 for this one).  Returns grid +
// the count before the claim (>= rows: nothing left).  The first claim of a
// call installs its tag (compare-and-swap); every later one is a single
// fetch-and-add, which the device serves back to back, where a
// compare-and-swap loop lets one claim through per round trip to memory
// (with rows of some 40 us, the workgroups then queued for their claims).
// The count stays below 2^24: at most rows + grid claims.
__device__ __noinline__ int claim_row(unsigned long long* word, unsigned long long epoch, int grid) {
  constexpr unsigned long long kCnt = (1ull << 24) - 1;
  const unsigned long long tag = (epoch & ((1ull << 40) - 1)) << 24;
  unsigned long long old = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (;;) {
    if ((old & ~kCnt) == tag) {
      const unsigned long long prev = __hip_atomic_fetch_add(word, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return grid + (int)(prev & kCnt);
    }
    unsigned long long expected = old;
    if (__hip_atomic_compare_exchange_strong(word, &expected, tag | 1ull, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT))
      return grid;
    old = expected;
  }
}

// FASTLD: 16-byte aligned rows with n % 4 == 0 (one float4 per lane per
// segment through buffer loads); otherwise element loads.  XF: the rows are
// read through post-processing and/or the fused repetition penalty
// (llz_xform.h); otherwise as they are.
// wslot: the workgroup's block of the special-queue overflow area.
template <bool FASTLD, int XM, bool EXT = false>
__device__ __forceinline__ void stats_row(const KArgs& A, int row, StatsShared& U, PenShared& pen_sh, int wslot) {
  constexpr bool XF = XM != kXmNone;
  const RowParams P = A.P;
  const RowPtrs Q = A.Q;
  constexpr int dcap = DCAP;  // EXACT slots per round
  FastShared& F = U.fast;
  LLZ_STAMP(row, 0);
  const int t = (int)threadIdx.x, lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(wave_id());  // wave-uniform: scalar registers
  const int n = P.n;
  const bool t1 = (P.flags & kFlagTIsOne) != 0;
  const float* xr = Q.src + (int64_t)row * P.src_stride;
  // reads of the row through the caller's post-processing and the penalty
  // (plain reads when !XF)
  using Src = typename std::conditional<XM == kXmCap, RowSrc,
                                        typename std::conditional<XF, LightSrc, PlainSrc>::type>::type;
  using OSrc = typename std::conditional<XF, RowSrc, PlainSrc>::type;
  Src X;   // the chain's input
  OSrc O;  // sampleArgmax's input (sampler.zig:89)
  if constexpr (XF) {
    X = row_src<XM == kXmCap>(P, Q, row, &pen_sh);
    O = row_orig(P, Q, row);
  } else {
    X = PlainSrc{xr};
    O = PlainSrc{Q.orig + (int64_t)row * P.orig_stride};
  }
  uint64_t pen_wm = 0;  // segments of this wave holding a penalised position
  // the penalty window's ids, loaded now by every wave (lane j: id j): the
  // penalty is applied after the load loop, which does not need it, so the
  // load lands meanwhile
  uint32_t pen_id = 0xffffffffu;
  if constexpr (XF) {
    if (P.xf_src & kXfPen) pen_id = pen_window_id(P, Q, row);
  }
  // Phase L's per-element work is the plain rows' plus, at most, one
  // multiply (kXmLight: the logit scale; 1 without one, v * 1 == v) or the
  // soft-cap estimate (kXmCap: cap_est on the raw logit, after the raw
  // maximum has taken it).  The penalty is applied to the few elements it
  // touches after the loop (the loop holds the row's register segments and
  // six loads in flight: any code that branches on the penalty inside it
  // costs registers it does not have).
  const float xscale = (XM == kXmLight && (P.xf_src & kXfScale)) ? P.inv_scale : 1.0f;
  auto seg_in = [&](const int k, float4 v) -> float4 {
    if constexpr (XM == kXmLight) {
      const int pos = (w + W * k) * SEG + lane * 4;
      v.x = (FASTLD || pos + 0 < n) ? v.x * xscale : v.x;
      v.y = (FASTLD || pos + 1 < n) ? v.y * xscale : v.y;
      v.z = (FASTLD || pos + 2 < n) ? v.z * xscale : v.z;
      v.w = (FASTLD || pos + 3 < n) ? v.w * xscale : v.w;
    }
    return v;
  };
  // the estimate's source value of a maximum-source value v (kXmCap: its
  // soft-cap estimate)
  auto est_of = [&](float v) -> float {
    if constexpr (XM == kXmCap) return cap_est(v, P.cap_a2, P.cap_c);
    return v;
  };
  const float l2e_t = P.l2e_t;
  const int G = (n + SEG - 1) / SEG;
  const int SPW = (G + W - 1) / W;
  const bool fits = SPW <= SPWMAX && P.cand_theta > 0.0f && fabsf(l2e_t) <= 0x1p40f && !(P.flags & kFlagXfExact);
  // the row's uniform, read now: the selection stage's draw needs it at the
  // end of a long serial path (a memory barrier keeps the load here)
  const float u_row = Q.uniforms[row];
  // wave w owns segments w, w + W, w + 2W, ...: its k-th is segment w + W k
  // (interleaved, so the costly start of the row is shared by every wave)
  const int nseg_w = fits ? max(0, (G - w + W - 1) / W) : 0;
  const int base_w = w * SEG + lane * 4;
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (kWave - lane));

  // ---- phase L: per segment as it lands: running maximum, the estimate q
  // (stored over v) and the segment sum of q (lane 63 stores it)
  float4 d[KV];
  float mx = -kInfS, cw = 0.0f;
  uint32_t nanf = 0;
  const int lane4 = lane * 4;
  const int lim_w = nseg_w > 0 ? n - w * SEG : 0;  // segment k holds positions lane4 < lim_w - k W SEG
  // bounds as (lane offset, VGPR) < (scalar limit of the segment); the
  // limits are recomputed in place (an empty asm keeps the compiler from
  // hoisting them all into live registers)
  auto seg_lim = [&](int k) {
    int l = k < nseg_w ? lim_w - k * (W * SEG) : 0;
    asm volatile("" : "+s"(l));
    return l;
  };
  // one segment's estimate: positions outside the row or the wave's segments
  // get an infinite offset, so q = 0, and no part in the maximum.  The
  // maximum takes the logits as they are (max3_raw: a signalling NaN makes it
  // NaN; its segment sum is NaN too, and phase M redoes such a row's maximum)
  auto seg_q = [&](const int k, float4 v) {
    const bool ok = lane4 < seg_lim(k);
    const float ck = ok ? cw : kInfS;
    if constexpr (XM != kXmCap) {  // kXmCap: the maximum comes from the estimates after the loop
      const float m = max3_raw(max3_raw(mx, v.x, v.y), v.z, v.w);
      mx = ok ? m : mx;
    }
    if constexpr (XM == kXmCap) {  // in place
      v.x = est_of(v.x);
      v.y = est_of(v.y);
      v.z = est_of(v.z);
      v.w = est_of(v.w);
      if constexpr (!FASTLD) {  // single positions past the row: no estimate (q = 0)
        const int pos = (w + W * k) * SEG + lane4;
        v.x = pos + 0 < n ? v.x : -kInfS;
        v.y = pos + 1 < n ? v.y : -kInfS;
        v.z = pos + 2 < n ? v.z : -kInfS;
        v.w = pos + 3 < n ? v.w : -kInfS;
      }
    }
    return q_of(v, l2e_t, ck);
  };
  // segment sums: lane k of my_a holds segment k's (stored after the loop)
  float my_a = 0.0f;
  auto seg_sum = [&](const int k, float4 q) {
    const float a = wave_fold_f32((q.x + q.y) + (q.z + q.w));
    my_a = __int_as_float(llz_writelane_i32(__builtin_amdgcn_readlane(__float_as_int(a), kWave - 1), k, __float_as_int(my_a)));
  };
  auto set_cw = [&](float mr) {
    // any finite reference of this wave: |m - mr| is checked in phase M
    if (!(fabsf(mr) <= 3.0e38f)) mr = 0.0f;
    cw = mr * l2e_t;
  };
  if constexpr (FASTLD) {
    // A window of kLoadWindow loads in flight per wave, one issued as each
    // segment is done: each CU's share of HBM arrives spread over the whole
    // read, and each segment's work overlaps the loads behind it (with every
    // load issued at once, a CU's data lands in one burst and the work
    // follows it).  Issue order = processing order: the LDS-resident segments
    // KV .. SPWMAX - 1 first (straight to LDS), then the register segments
    // 0 .. KV - 1.  Every slot issues exactly one load (reads past the row
    // return zeros), so the wait for slot i counts the loads behind it.
    const llz_i4v rs = row_rsrc(xr, (uint32_t)n * 4u);
    const int soff = __builtin_amdgcn_readfirstlane(w * SEG * 4);
    const uint32_t lds0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uintptr_t)&F.u.data[w][0][0]);
    auto issue = [&](const int i) {
      if (i < KL)
        dma_buf16(rs, lane * 16, soff + (KV + i) * (W * SEG * 4), lds0 + (uint32_t)(i * SEG * 4));
      else
        d[i - KL] = buf_ld4(rs, lane * 16, soff + (i - KL) * (W * SEG * 4));
      __builtin_amdgcn_sched_barrier(0);  // keep the issue order
    };
    static_assert(kLoadWindow >= 1 && kLoadWindow <= KV, "a full window behind every LDS-resident segment");
#pragma unroll
    for (int i = 0; i < kLoadWindow; ++i) issue(i);
#pragma unroll
    for (int i = 0; i < SPWMAX; ++i) {
      if (i < KL) {
        const int k = KV + i;
        if (k < nseg_w) {
          lds_dma_wait<kLoadWindow - 1>();  // the window's loads behind it (the register ones come later)
          float4* p = reinterpret_cast<float4*>(&F.u.data[w][i][lane * 4]);
          const float4 v = seg_in(k, *p);
          if (i == 0) set_cw(wave_max_f32(lane4 < seg_lim(k) ? est_of(max4(v)) : -kInfS));  // the first segment processed
          const float4 q = seg_q(k, v);
          *p = q;
          seg_sum(k, q);
        }
      } else {
        const int k = i - KL;
        const float4 v = seg_in(k, d[k]);
        if (k == 0 && nseg_w <= KV) set_cw(wave_max_f32(lane4 < seg_lim(0) ? est_of(max4(v)) : -kInfS));
        float4 q = seg_q(k, v);  // a NaN logit makes its segment sum NaN
        // materialise q here, while the loads land (not sunk into phase S)
        asm volatile("" : "+v"(q.x), "+v"(q.y), "+v"(q.z), "+v"(q.w));
        d[k] = q;
        seg_sum(k, q);
      }
      // (issue() ends with a scheduling barrier: segments stay in order while
      // loads are issued; the last kLoadWindow may interleave)
      if (i + kLoadWindow < SPWMAX) issue(i + kLoadWindow);
    }
  } else {
    // element loads, all in flight at once (guarded loads are waited for
    // where they are read)
#pragma unroll
    for (int k = 0; k < KV; ++k) d[k] = ld1x4(xr, base_w + k * (W * SEG), k < nseg_w ? n : 0);
    for (int k = KV; k < nseg_w; ++k) seg_to_lds(xr, w + W * k, n, false, &F.u.data[w][k - KV][0]);
    __builtin_amdgcn_sched_barrier(0);
    const float4 v0 = seg_in(0, d[0]);
    set_cw(wave_max_f32(lane4 < seg_lim(0) ? est_of(max4(v0)) : -kInfS));
#pragma unroll
    for (int k = 0; k < KV; ++k) {
      float4 v = v0;
      if (k > 0) v = seg_in(k, d[k]);
      float4 q = seg_q(k, v);
      asm volatile("" : "+v"(q.x), "+v"(q.y), "+v"(q.z), "+v"(q.w));
      d[k] = q;
      seg_sum(k, q);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int k = KV; k < nseg_w; ++k) {
      float4* p = reinterpret_cast<float4*>(&F.u.data[w][k - KV][lane * 4]);
      const float4 q = seg_q(k, seg_in(k, *p));
      *p = q;
      seg_sum(k, q);
    }
  }
  // ---- the penalty (sampler.zig:54-75) on this wave's penalised elements,
  // after the loop.  Lane j takes the row's penalised position j when it lies
  // in one of this wave's segments: it reads the logit, and the element's
  // estimate becomes the one phase L would have computed for the penalised
  // value (kXmLight: penalise(v s), exact; kXmCap: pen_est of the soft-cap
  // estimate); each touched segment's sum of estimates is folded again as
  // phase L folds it.  LDS-resident segments take the estimate from the lane
  // that holds the position, register segments from the lane that owns it.
  LLZ_STAMP(row, 46);
  uint32_t pen_p = 0xffffffffu;  // this lane's penalised position (of this wave's segments)
  float pen_r = 0.0f;            // its logit as the caller wrote it
  uint64_t pen_lanes = 0ull;     // the lanes holding one
  uint32_t pen_idf = 0xffffffffu;  // lane j: id j, bit 31 set unless its first occurrence of an id < n
  if constexpr (XF) {
    if (P.xf_src & kXfPen) {
      // Each wave takes the window's distinct ids < n (sampler.zig:62-70
      // penalises an id once) in its own segments from its registers: no
      // barrier waits for the other waves here.
      bool first = pen_id < (uint32_t)n;
      for (int j = 0; j < P.pen_w; ++j) {
        const uint32_t o = readlane_u32(pen_id, j);
        first = first && !(j < lane && o == pen_id);
      }
      pen_idf = first ? pen_id : (pen_id | 0x80000000u);
      const bool mine = first && ((pen_id >> 8) & (uint32_t)(W - 1)) == (uint32_t)w;
      pen_p = mine ? pen_id : 0xffffffffu;
      pen_r = mine ? xr[pen_id] : 0.0f;
      pen_lanes = bal64(mine);
      for (uint64_t bm = pen_lanes; bm != 0ull; bm &= bm - 1ull) {
        const uint32_t k = readlane_u32(pen_id, __ffsll((long long)bm) - 1) >> 11;  // segment pos >> 8 = w + W k
        if (k < 64u) pen_wm |= 1ull << k;
      }
    }
    if (fits && pen_wm != 0ull) {
      const uint32_t pp = pen_p;
      const bool mine = pp != 0xffffffffu;
      const float src = XM == kXmCap ? pen_est(est_of(pen_r), P.rpen, P.rpen_inv) : penalise(pen_r * xscale, P.rpen);
      const float qn = __builtin_amdgcn_exp2f(fmaf(src, l2e_t, -cw));
      const int kk = (int)(pp >> 11);  // the wave's segment index k of segment pp >> 8 = w + W k
      if (mine && kk >= KV) F.u.data[w][kk - KV][pp & (uint32_t)(SEG - 1)] = qn;
#pragma unroll
      for (int k = 0; k < KV; ++k) {
        if ((pen_wm >> k) & 1ull) {
          uint64_t bm = bal64(mine && kk == k);
          while (bm != 0ull) {
            const int b = __ffsll((long long)bm) - 1;
            bm &= bm - 1ull;
            const uint32_t pb = readlane_u32(pp, b);
            const float qb = __uint_as_float(readlane_u32(__float_as_uint(qn), b));
            const uint32_t c = pb & 3u;
            const bool own = (uint32_t)lane == ((pb >> 2) & 63u);
            d[k].x = own && c == 0u ? qb : d[k].x;
            d[k].y = own && c == 1u ? qb : d[k].y;
            d[k].z = own && c == 2u ? qb : d[k].z;
            d[k].w = own && c == 3u ? qb : d[k].w;
          }
          seg_sum(k, d[k]);
        }
      }
      __builtin_amdgcn_wave_barrier();  // this wave's own LDS writes: LDS order suffices
      for (uint64_t rest = pen_wm >> KV; rest != 0ull; rest &= rest - 1ull) {
        const int k = KV + __ffsll((long long)rest) - 1;
        seg_sum(k, *reinterpret_cast<const float4*>(&F.u.data[w][k - KV][lane * 4]));
      }
      LLZ_STAMP(row, 44);
    }
  }
  // a position of this wave's segments through the row's transforms,
  // exactly, the penalty from the wave's own list (the shared one is built
  // below, read after the next barrier)
  auto fix_here = [&](int pos, float v) -> float {
    if constexpr (!XF) {
      return v;
    } else {
      v = X.pre(v);
      bool hit = false;
      if ((pen_wm >> (((uint32_t)pos >> 11) & 63u)) & 1ull) {  // a segment holding one (most hold none)
        for (uint64_t bm = pen_lanes; bm != 0ull; bm &= bm - 1ull)
          hit = hit || (uint32_t)pos == readlane_u32(pen_p, __ffsll((long long)bm) - 1);
      }
      return hit ? penalise(v, P.rpen) : v;
    }
  };
  if constexpr (XF) {
    // the row's sorted list of penalised positions and the waves' segment
    // masks in LDS (wave 0): the rows the single pass does not take read it
    // in their scan right below; the others only if they go on to the exact
    // phases (built there: a row the token path finishes never needs it)
    if ((P.xf_src & kXfPen) && !fits) {
      pen_list(pen_sh, pen_idf);
      lds_barrier();
    }
  }
  if (lane < nseg_w) F.v.aseg[w + W * lane] = my_a;
  // token-only calls: this wave's sum of its estimates (the normaliser's
  // estimate in phase M takes one value per wave)
  const bool tok = (P.flags & kFlagTokenOnly) != 0u && fits;
  if (tok) {
    const float qs = wave_fold_f32(lane < nseg_w ? my_a : 0.0f);
    // and weighted by where they lie: segment w + W lane starts at position
    // SEG (w + W lane), so each of its terms' weight n - pos is at most
    // n - SEG (w + W lane) (the interval of S in llz_token.h)
    const float qw = wave_fold_f32(lane < nseg_w ? my_a * (float)(n - SEG * (w + W * lane)) : 0.0f);
    if (lane == kWave - 1) {
      F.qsum[w] = qs;
      F.qwsum[w] = qw;
    }
  }
  if (!fits) {  // rows the fast path does not take: maximum and NaN scan only
    if constexpr (FASTLD) {
      // kScanDepth float4 loads per thread in flight (64 KB per workgroup)
      constexpr int U = kScanDepth;
      for (int b = t * 4; b < n; b += NT * 4 * U) {
        float4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = ld4(xr, b + u * (NT * 4), n);  // absent: -inf
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float4 f = X.fix4(b + u * (NT * 4), v[u], n);
          mx = fmaxf(mx, max4(f));  // fmaxf skips NaN, as the scalar loop did
          nanf |= (uint32_t)((f.x != f.x) | (f.y != f.y) | (f.z != f.z) | (f.w != f.w));
        }
      }
    } else {
      for (int i = t; i < n; i += NT) {
        const float v = X.at(i);
        mx = fmaxf(mx, v);
        nanf |= (uint32_t)(v != v);
      }
    }
  }
  mx = wave_max_f32(mx);
  if constexpr (XF) {
    if (fits) {
      // The wave's exact maximum from the estimates as they stand (penalised
      // elements patched): an element of the largest value has the largest
      // term, and every estimate lies within eps of its term (2^-16 on the
      // scaled rows, 2^-16 + est_xe <= 2^-10.9 on soft-capped ones), so its
      // q >= q_max (1 - eps) / (1 + eps) >= q_max (1 - 2^-9); each lane's
      // segments holding such an estimate are read again and evaluated
      // exactly.  (Nothing here takes f(max) for max(f): tanh_f32, like the
      // reference's tanhf, is not monotone between adjacent floats.)
      auto scan_max = [&]() -> float {
        float ql = 0.0f;
#pragma unroll
        for (int k = 0; k < KV; ++k) ql = fmaxf(ql, max4(d[k]));  // absent lanes and segments hold q = 0
        for (int k = KV; k < nseg_w; ++k) ql = fmaxf(ql, max4(*reinterpret_cast<const float4*>(&F.u.data[w][k - KV][lane * 4])));
        const float qthr = wave_max_f32(ql) * (1.0f - 0x1p-9f);
        uint64_t sm = 0ull;
#pragma unroll
        for (int k = 0; k < KV; ++k) sm |= (max4(d[k]) >= qthr ? 1ull : 0ull) << k;
        for (int k = KV; k < nseg_w; ++k)
          sm |= (max4(*reinterpret_cast<const float4*>(&F.u.data[w][k - KV][lane * 4])) >= qthr ? 1ull : 0ull) << k;
        float ex = -kInfS;
        while (sm != 0ull) {
          const int k = __ffsll((long long)sm) - 1;
          sm &= sm - 1ull;
          const int pos = (w + W * k) * SEG + lane4;
#pragma unroll 1
          for (int c = 0; c < 4; ++c)
            if (pos + c < n) ex = fmaxf(ex, fix_here(pos + c, xr[pos + c]));
        }
        return wave_max_f32(ex);
      };
      if constexpr (XM == kXmCap) {
        // phase L took no maximum (the soft-cap's exact value costs some
        // sixty operations; the estimates locate the largest elements)
        mx = scan_max();
      } else if (pen_wm != 0ull) {
        // phase L's maximum is that of the scaled logits, the penalised
        // ones at their unpenalised values: when none of those held it, the
        // others' maximum stands and the penalised values join it
        const bool mine = pen_p != 0xffffffffu;
        const bool top = bal64(mine && pen_r * xscale == mx) != 0ull;
        mx = top ? scan_max() : fmaxf(mx, wave_max_f32(mine ? penalise(X.pre(pen_r), P.rpen) : -kInfS));
      }
      LLZ_STAMP(row, 45);
    }
  }
  // token-only rows: the lanes that may hold a candidate (a term that may
  // reach thr_e; Rw scales this wave's estimates q to terms), queued in
  // F.qpos[w] and re-read into tv.  The segments whose estimated sum reaches
  // thr_e, then their lanes holding an estimate that does (estimates are
  // within 2^-16 of the terms, no term exceeds its segment's sum, positions
  // outside the row hold q = 0).  Returns the number of lanes found; none
  // beyond QCAP is re-read.
  float4 tv[QCAP / kWave];
  auto tqueue = [&](const float Rw, const float thr_e) -> int {
    const uint64_t segm = bal64(lane < nseg_w && my_a * Rw >= thr_e);
    const float thr_q = thr_e / Rw;
    // the lane's candidate segments as a bit mask: the register segments
    // without a branch, the LDS-resident ones where the segment's sum passes
    uint32_t lm_lo = 0u, lm_hi = 0u;
    auto tflag = [&](const int k, const float4 q) {
      const uint32_t c = max3_raw(max3_raw(q.x, q.y, q.z), q.w, q.w) >= thr_q ? 1u : 0u;
      if (k < 32)
        lm_lo |= c << k;
      else
        lm_hi |= c << (k - 32);
    };
#pragma unroll
    for (int k = 0; k < KV; ++k) tflag(k, d[k]);
    for (uint64_t rest = segm >> KV; rest != 0ull; rest &= rest - 1ull) {
      const int k = KV + __ffsll((long long)rest) - 1;
      const float4 q = *reinterpret_cast<const float4*>(&F.u.data[w][k - KV][lane * 4]);
      const uint32_t c = max3_raw(max3_raw(q.x, q.y, q.z), q.w, q.w) >= thr_q ? 1u : 0u;
      lm_hi |= c << (k - 32);  // k >= KV > 32
    }
    uint64_t lm = ((uint64_t)lm_hi << 32) | lm_lo;
    const uint32_t nb = (uint32_t)__popcll(lm);
    const uint32_t nb_in = wave_incl_scan_op(nb, 0u, [](uint32_t a, uint32_t b) { return a + b; });
    const int nq = (int)readlane_u32(nb_in, kWave - 1);
    for (uint32_t slot = nb_in - nb; lm != 0ull; lm &= lm - 1ull, ++slot) {
      const int k = __ffsll((long long)lm) - 1;
      if (slot < (uint32_t)QCAP) F.qpos[w][slot] = (uint32_t)((w + W * k) * SEG + lane4);
    }
    __builtin_amdgcn_wave_barrier();  // this wave's own queue: LDS order suffices
    // an overflowing queue fails the row: no re-reads for it
    if (nq <= QCAP) {
#pragma unroll
      for (int h = 0; h < QCAP / kWave; ++h) {
        const int i = h * kWave + lane;
        const int pos = i < nq ? (int)F.qpos[w][i] : 0;
        tv[h] = FASTLD ? ld4(xr, pos, n) : ld1x4(xr, pos, n);  // raw: transformed where they are read
      }
    } else {
#pragma unroll
      for (int h = 0; h < QCAP / kWave; ++h) tv[h] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    return nq;
  };
  // queued now against this wave's own maximum (m >= mx, so a superset of
  // the lanes against the row's; the threshold lowered by 2^-12 more covers
  // the roundings of R), the re-reads in flight while the other waves finish
  // their loads; a wave whose superset overflows the queue scans again
  // against the row's maximum after the barrier
  int tq = -1;
  if (tok && l2e_t > 0.0f) {
    const float aw = fmaf(mx, -l2e_t, cw);
    if (fabsf(aw) <= 64.0f) {
      const int q0 = tqueue(__builtin_amdgcn_exp2f(aw), P.tok_theta * (1.0f - 0x1p-10f) * (1.0f - 0x1p-12f));
      if (q0 <= QCAP) tq = q0;
    }
  }
  const bool wnan = bal64(nanf != 0u) != 0ull;
  if (lane == 0) {
    F.mw[w] = mx;
    F.cw[w] = cw;
    F.nanw[w] = wnan ? 1u : 0u;
  }
  if (t == 0) {
    F.fail = fits ? 0u : 1u;
    F.flood = 0;
    F.ncand = 0;
    F.nslot = 1;  // slot 0 is the row's first segment's
    F.slotseg[0] = 0;
    F.next_e = 0;
    F.s_run = 0.0f;
    F.done = 0;
    F.diag = 0;
    F.tcand = 0u;  // the token-only list (ordered before its atomics by the barrier below)
    F.tfail = 0u;
  }
  if constexpr (FASTLD) {
    // every load of the row has landed (the register segments, issued after
    // the LDS-resident ones, were consumed): the barrier orders LDS only, and
    // a token-only row's re-reads stay in flight across it
    lds_barrier();
  } else {
    __syncthreads();
  }
  LLZ_STAMP(row, 1);

  // ---- phase M: row maximum, scale factors, binade prediction, first slots
  float m = -kInfS;
  bool nanrow = false;
#pragma unroll
  for (int i = 0; i < W; ++i) {
    m = fmaxf(m, F.mw[i]);
    nanrow = nanrow | (F.nanw[i] != 0u);
  }
  // ---- token-only rows (no probabilities or statistics asked for, no
  // typical-p): the chain's decisions from the candidates' exact terms and an
  // interval for the normaliser (token_select), without the rest of phase M
  // and phases S .. C.  The normaliser's estimate: the waves' sums of
  // estimates, each scaled by its R.  Candidates: the lanes of segments
  // whose estimated sum reaches theta (1 - 2^-10) holding a term whose
  // estimate does (estimates are within 2^-16 of the terms, and no term
  // exceeds its segment's sum), re-read and evaluated exactly; the list lies
  // in F.v, free once every wave has read the segment sums below.
  if (tok && !nanrow && fabsf(m) <= 3.0e38f && P.tok_theta > 0.0f) {
    LLZ_STAMP(row, 38);
    float s_est = 0.0f, w_est = 0.0f;
    bool tbad = false;
#pragma unroll
    for (int i = 0; i < W; ++i) {
      const float awi = fmaf(m, -l2e_t, F.cw[i]);
      tbad = tbad | ((G > i) & !(fabsf(awi) <= 64.0f));
      const float ri = __builtin_amdgcn_exp2f(awi);
      s_est += G > i ? F.qsum[i] * ri : 0.0f;
      w_est += G > i ? F.qwsum[i] * ri : 0.0f;
    }
    // (soft-capped rows leave typical-p to the exact phases: the register
    // pressure of its code spilled in the capped kernel's token path)
    const bool typ = EXT && XM != kXmCap && P.typical_p > 0.0f && P.typical_p < 1.0f;
    if (!tbad && typ) {
      // typical-p (sampler.zig:128-132): this wave's part of sum_i e_i log2
      // e_i, from its estimates (e_i ~ q_i R_w, log2 e_i ~ log2 q_i + aw),
      // and the sum of the parts' magnitudes for the error bound.  Every
      // position outside the row or the wave's segments has q = 0; the
      // segments past the wave's last are not read
      const float aw = fmaf(m, -l2e_t, cw);
      float sx = 0.0f, sa = 0.0f;
      auto acc = [&](float q) {
        const float y = q >= 0x1p-100f ? q * (__builtin_amdgcn_logf(q) + aw) : 0.0f;
        sx += y;
        sa += fabsf(y);
      };
#pragma unroll
      for (int k = 0; k < KV; ++k) {
        acc(d[k].x);
        acc(d[k].y);
        acc(d[k].z);
        acc(d[k].w);
      }
      for (int i = 0; i < KL && KV + i < nseg_w; ++i) {
        const float4 q = *reinterpret_cast<const float4*>(&F.u.data[w][i][lane * 4]);
        acc(q.x);
        acc(q.y);
        acc(q.z);
        acc(q.w);
      }
      sx = wave_sum_f32(sx);
      sa = wave_sum_f32(sa);
      if (lane == 0) {
        F.tx[w] = sx;
        F.txa[w] = sa;
      }
    }
    if (!tbad) {
      const float Rw_t = __builtin_amdgcn_exp2f(fmaf(m, -l2e_t, cw));
      uint64_t* const tl = reinterpret_cast<uint64_t*>(&F.v);  // [kTokCap] collected, then [kTokCap] sorted
      static_assert(sizeof(F.qpos) >= (size_t)(kNT / kWave) * kTokCap * sizeof(uint8_t), "partial ranks fit the queue rows");
      static_assert(sizeof(F.v) >= 2 * kTokCap * sizeof(uint64_t), "the list and its sorted copy fit F.v");
      // Round 0 collects the terms e >= tok_theta.  A list that overflows
      // under a top-k of at most kTokCap / 4 is collected again (round 1)
      // above theta2: just below the (top_k + 1)-th largest of the terms
      // collected (a subset's order statistic, at most the row's), so the
      // top_k + 1 largest terms lie clear above it
      auto collect = [&](const float theta_t) {
      const float thr_e = theta_t * (1.0f - 0x1p-10f);
      if (tq < 0) tq = tqueue(Rw_t, thr_e);
      LLZ_STAMP(row, 39);
      LLZ_STAMP(row, 32);
      if (tq > QCAP && lane == 0) atomicOr(&F.tfail, 1u);
      // The queued lanes' elements that may be candidates: the lane test
      // (tqueue against the row's maximum) element by element, on the same
      // estimates exp2(fma(v, l2e_t, -cw)) phase L computed.  When a wave
      // has at most 64 of them, they are staged in its queue row as (logit,
      // position) pairs and each lane evaluates one exact term; one LDS
      // atomic per wave reserves its list slots.  Otherwise every queued
      // lane evaluates its four terms.
      constexpr int NH = QCAP / kWave;
      int tpos[NH];
      uint32_t tmk[NH];
      uint32_t tcnt = 0u;
      const float thr_q = thr_e / Rw_t;
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        const int i = h * kWave + lane;
        const bool live = tq <= QCAP && i < tq;
        tpos[h] = live ? (int)F.qpos[w][i] : 0;
        // the re-reads as the chain reads them (kXmLight: exactly; kXmCap
        // keeps them raw: its test below takes estimates, and the exact
        // values are taken for the candidates alone)
        if constexpr (XM == kXmLight) {
          tv[h].x = fix_here(tpos[h] + 0, tv[h].x);
          tv[h].y = fix_here(tpos[h] + 1, tv[h].y);
          tv[h].z = fix_here(tpos[h] + 2, tv[h].z);
          tv[h].w = fix_here(tpos[h] + 3, tv[h].w);
        }
        const float vs[4] = {tv[h].x, tv[h].y, tv[h].z, tv[h].w};
        uint32_t mk = 0u;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          // kXmCap: the element's estimate (soft-cap, and the penalty where it
          // applies), within 2^-16 + est_xe <= 2^-10.9 of the term, inside
          // thr_e's margin of 2^-10
          float vq = vs[c];
          if constexpr (XM == kXmCap) {
            vq = est_of(vq);
            bool hit = false;  // a penalised position of this wave's
            if ((pen_wm >> (((uint32_t)(tpos[h] + c) >> 11) & 63u)) & 1ull) {
              for (uint64_t bm = pen_lanes; bm != 0ull; bm &= bm - 1ull)
                hit = hit || (uint32_t)(tpos[h] + c) == readlane_u32(pen_p, __ffsll((long long)bm) - 1);
            }
            if (hit) vq = pen_est(vq, P.rpen, P.rpen_inv);
          }
          const bool pass = live && tpos[h] + c < n && __builtin_amdgcn_exp2f(fmaf(vq, l2e_t, -cw)) >= thr_q;
          mk |= pass ? (1u << c) : 0u;
        }
        tmk[h] = mk;
        tcnt += (uint32_t)__popc(mk);
      }
      const uint32_t tinc = wave_incl_scan_op(tcnt, 0u, [](uint32_t a, uint32_t b) { return a + b; });
      const int ttot = (int)readlane_u32(tinc, kWave - 1);
      if (ttot <= kWave) {
        uint32_t* const sg = &F.qpos[w][0];  // [64][2]: this wave's row, read above (LDS order suffices)
        __builtin_amdgcn_wave_barrier();
        uint32_t o = tinc - tcnt;
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          const float vs[4] = {tv[h].x, tv[h].y, tv[h].z, tv[h].w};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            if ((tmk[h] >> c) & 1u) {
              sg[2 * o] = __float_as_uint(vs[c]);
              sg[2 * o + 1] = (uint32_t)(tpos[h] + c);
              ++o;
            }
          }
        }
        __builtin_amdgcn_wave_barrier();
        float e = 0.0f;
        uint32_t id = 0u;
        if (lane < ttot) {
          id = sg[2 * lane + 1];
          float v = __uint_as_float(sg[2 * lane]);
          if constexpr (XM == kXmCap) v = fix_here((int)id, v);  // the exact value of a raw re-read
          e = exact_term(v, m, P.temperature, t1);  // sampler.zig:85
        }
        const bool cand = lane < ttot && e >= theta_t;
        const uint64_t cb = bal64(cand);
        if (cb != 0ull) {
          uint32_t base = 0u;
          if (lane == 0) base = atomicAdd(&F.tcand, (uint32_t)__popcll(cb));
          base = readlane_u32(base, 0);
          const uint32_t slot = base + (uint32_t)__popcll(cb & lt_mask);
          if (cand && slot < (uint32_t)kTokCap) tl[slot] = ((uint64_t)(~__float_as_uint(e)) << 32) | id;
        }
      } else {
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          if (tmk[h] != 0u) {
            const int pos = tpos[h];
            float4 v4 = tv[h];
            if constexpr (XM == kXmCap) {
              v4.x = pos + 0 < n ? fix_here(pos + 0, v4.x) : v4.x;
              v4.y = pos + 1 < n ? fix_here(pos + 1, v4.y) : v4.y;
              v4.z = pos + 2 < n ? fix_here(pos + 2, v4.z) : v4.z;
              v4.w = pos + 3 < n ? fix_here(pos + 3, v4.w) : v4.w;
            }
            const float4 e = exact_terms4(v4, m, P.temperature, t1);  // sampler.zig:85
            const float es[4] = {e.x, e.y, e.z, e.w};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              if (pos + c < n && es[c] >= theta_t) {
                const uint32_t slot = atomicAdd(&F.tcand, 1u);
                if (slot < (uint32_t)kTokCap) tl[slot] = ((uint64_t)(~__float_as_uint(es[c])) << 32) | (uint32_t)(pos + c);
              }
            }
          }
        }
      }
      lds_barrier();  // the list complete (LDS only: the re-reads were consumed above)
      LLZ_STAMP(row, 33);
      };
      collect(P.tok_theta);
      float theta_t = P.tok_theta;
      const uint32_t kk = P.top_k;
      if (EXT && XM != kXmCap && F.tcand > (uint32_t)kTokCap && F.tfail == 0u && kk >= 1u && kk <= (uint32_t)(kTokCap / 4) &&
          kk < (uint32_t)n) {
        token_sort(tl, tl + kTokCap, reinterpret_cast<uint8_t*>(&F.qpos[0][0]), kTokCap);
        if (t == 0) {  // wave 0 placed the sorted keys
          const float e1 = __uint_as_float(~(uint32_t)(tl[kTokCap + kk] >> 32));
          F.theta2 = fmaxf(e1 * (1.0f - 0x1p-19f), P.tok_theta);
          F.tcand = 0u;
        }
        lds_barrier();
        theta_t = F.theta2;
        tq = -1;
        collect(theta_t);
      }
      const int tc = (int)F.tcand;
      if (tc <= kTokCap && F.tfail == 0u) {
        token_sort(tl, tl + kTokCap, reinterpret_cast<uint8_t*>(&F.qpos[0][0]), tc);
        LLZ_STAMP(row, 34);
        if (w == 0) {
          // typical-p rows take their own copy of the decisions, so that the
          // others keep the shorter chain
          if (typ) {
            double hs_lo = 0.0, hs_hi = -1.0;  // the row's entropy
            entropy_star(P, F.tx, F.txa, F.qsum, F.cw, W, G, m, s_est, &hs_lo, &hs_hi);
            token_select<true>(kernel_args_ptr(), row, tl + kTokCap, tc, s_est, w_est, hs_lo, hs_hi, u_row, theta_t,
                               &F.tfail);
          } else {
            token_select<false>(kernel_args_ptr(), row, tl + kTokCap, tc, s_est, w_est, 0.0, -1.0, u_row, theta_t,
                                &F.tfail);
          }
        }
      } else if (t == 0) {
        F.tfail = 1u;
      }
      // LDS only: the outputs' global stores need not land before the
      // workgroup ends
      lds_barrier();
      if (F.tfail == 0u) {
        LLZ_STAMP(row, 15);
        return;
      }
      // not certified: the exact phases, with the segment sums the list
      // overwrote written again (F.qpos is rewritten in phase S)
      if (lane < nseg_w) F.v.aseg[w + W * lane] = my_a;
      __syncthreads();
    }
  }
  if constexpr (XF) {
    if ((P.xf_src & kXfPen) && fits) {  // the exact phases read the list (see above)
      pen_list(pen_sh, pen_idf);
      LLZ_STAMP(row, 43);
      lds_barrier();
    }
  }
  // the segment sums of q of round `lane` (segments W lane .. W lane + W - 1,
  // one per wave), all read at once; absent ones are 0 (selects, not
  // branches: each branch here would wait out an LDS read of its own)
  float av[W];
  const int glast = min(G, GMAX) - 1;
#pragma unroll
  for (int i = 0; i < W; ++i) av[i] = F.v.aseg[min(W * lane + i, glast)];
#pragma unroll
  for (int i = 0; i < W; ++i) av[i] = W * lane + i < G ? av[i] : 0.0f;
  if (fits) {
    // a NaN logit makes its segment's sum of q NaN (q >= 0 otherwise, so
    // no inf - inf)
    bool nl = false;
#pragma unroll
    for (int i = 0; i < W; ++i) nl = nl | (av[i] != av[i]);
    if (bal64(nl) != 0ull) {
      // a NaN logit: phase L's maximum did not quiet signalling NaNs, so the
      // row's maximum is taken again (sampler.zig:80-81: NaNs are skipped)
      nanrow = true;
      float mm = -kInfS;
      for (int i = t; i < n; i += NT) mm = fmaxf(mm, X.at(i));
      mm = wave_max_f32(mm);
      __syncthreads();  // every wave has read F.mw
      if (lane == 0) F.mw[w] = mm;
      __syncthreads();
      m = -kInfS;
#pragma unroll
      for (int i = 0; i < W; ++i) m = fmaxf(m, F.mw[i]);
    }
  }
  // a NaN logit or an infinite maximum makes the reference's sum NaN: the
  // selection handles that row without the phases below
  const bool nan_sum = nanrow || !(fabsf(m) <= 3.0e38f);
  bool certified = true;
  float S = __builtin_nanf("");
  uint32_t cc = 0;
  bool pre_ok = false;     // candidates 0 .. cand_n0 - 1 are in cand_pre (read during the walk)
  uint64_t cand_pre = 0;
  uint32_t cand_n0 = 0;
  if (!nan_sum) {
    const float aw = fmaf(m, -l2e_t, cw);
    const float Rw = __builtin_amdgcn_exp2f(aw);  // q * Rw ~ e = exp((v - m) / T)
    if (lane == 0) F.bw[w] = fabsf(aw);
    // Prediction in index order: lane k takes round k (segments W k .. W k +
    // W - 1, one per wave, each scaled by its wave's R); a scan over the rounds
    // gives every segment's running sum.  Every wave computes it for its own
    // segments (the lane's segment of this wave is W k + w).
    const bool have = lane < nseg_w;
    {
      float rtot = 0.0f, before_w = 0.0f, b_w = 0.0f;
      bool bad = false;
      int gc = -1;  // the lane's last segment whose estimated sum is at least 1/2
#pragma unroll
      for (int i = 0; i < W; ++i) {
        const float awi = fmaf(m, -l2e_t, F.cw[i]);
        bad = bad | ((G > i) & !(fabsf(awi) <= 64.0f));
        const float ri = __builtin_amdgcn_exp2f(awi);
        const float b = W * lane + i < G ? av[i] * ri : 0.0f;
        rtot += b;
        before_w += i < w ? b : 0.0f;
        b_w = i == w ? b : b_w;
        gc = b >= 0.5f ? W * lane + i : gc;
      }
      // gm: the last segment whose estimated sum is at least 1/2.  The row's
      // maximum element has the term exp(0) = 1 exactly, estimated within a
      // tiny relative error, so its segment's estimate is above 1/2: the
      // maximum lies in segment gm or before.  The reference's running sum,
      // once it has added a term, is at least that term (RN(s + e) >= e for
      // s >= 0) and never decreases: after segment gm it is at least 1.
      // (lane k holds round k's segments, so the highest lane with one holds gm)
      const uint64_t cm = bal64(gc >= 0);
      const int gm = cm != 0ull ? (int)readlane_u32((uint32_t)gc, 63 - __builtin_clzll(cm)) : -1;
      const float rin = wave_incl_scan_f32(rtot);
      const float rex = __uint_as_float(wave_shift_up1(__float_as_uint(rin)));
      const float total = __uint_as_float(lane_readlast(__float_as_uint(rin)));
      bad = bad || !(total <= 3.0e38f);
      bool ex = false, fl = false;
      if (!bad && have) {
        const float excl = rex + before_w;
        const float incl = excl + b_w;
        // the prediction's lower end, raised to 1 after the maximum's segment
        // (a sum of 1 plus small terms would otherwise straddle 1 for the
        // rest of the row)
        const float lo = gm >= 0 && w + W * lane > gm ? fmaxf(excl * (1.0f - DELTA), 1.0f) : excl * (1.0f - DELTA);
        const float hi = incl * (1.0f + DELTA);
        const int elo = (int)(__float_as_uint(lo) >> 23) - 127;
        const int ehi = (int)(__float_as_uint(hi) >> 23) - 127;
        const bool plain = lo >= 0x1p-64f && hi <= 3.0e38f && elo == ehi;
        fl = plain && ldexpf(P.cand_theta, 23 - elo) < 2.0f;
        // EXACT: tabulate the binades from the one the segment starts in to
        // the one it ends in (the row's first segment starts at 0: its NG
        // highest, below them it is summed term by term)
        int j0 = lo >= 0x1p-126f ? elo : ehi - (NG - 1);
        j0 = max(-126, min(j0, 126));
        const int g = w + W * lane;
        F.sflag[g] = plain ? PLAIN : EXACT_PRED;
        F.sj[g] = (int8_t)(plain ? elo : j0);
        F.sng[g] = (uint8_t)max(1, min(ehi - j0 + 1, NG));
        ex = !plain;
      }
      // EXACT slots: 0 for the row's first segment (always EXACT: it starts at
      // 0), the others in any order from 1 (a row with more than DCAP takes
      // further rounds in index order)
      const uint64_t exm = bal64(ex) & (w == 0 ? ~1ull : ~0ull);
      int base = 0;
      if (lane == 0) {
        if (exm != 0ull) base = (int)atomicAdd((uint32_t*)&F.nslot, (uint32_t)__popcll(exm));
        if (bad) atomicOr(&F.fail, 1u);
        if (bal64(fl) != 0ull) atomicOr(&F.flood, 1u);
      }
      base = __builtin_amdgcn_readfirstlane(base);
      if (have) {
        const int slot = (w == 0 && lane == 0) ? 0 : base + __popcll(exm & lt_mask);
        const bool got = ex && slot < dcap;
        F.sdump[w + W * lane] = (int8_t)(got ? slot : -1);
        if (got) F.slotseg[slot] = (int16_t)(w + W * lane);
      }
    }
    __syncthreads();
    LLZ_STAMP(row, 2);
    const bool flood = F.flood != 0u;
    const float theta = flood ? kInfS : P.cand_theta;

    // ---- phase S: integer sums of PLAIN segments, four segments per step.
    // A lane whose roundings a segment cannot certify (its lower and upper
    // bracket sums differ, or a term reaches tspec: large terms and
    // candidates) is queued as the position of its first term and the parity
    // of the segment's integer sum before it; the queue is settled in phase
    // F+X.
    int qn = 0;
    float4 v4q[2];
    auto reread = [&](int cnt) {  // the logits of the first cnt queued lanes (wave-uniform)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int i = h * kWave + lane;
        const int pos = i < cnt ? (int)(F.qpos[w][i] & 0x7fffffffu) : 0;
        const float4 r = FASTLD ? ld4(xr, pos, n) : ld1x4(xr, pos, n);
        v4q[h] = XM == kXmCap ? r : X.fix4(pos, r, n);  // kXmCap: raw (settle_specials transforms them)
      }
    };
    auto settle = [&](int cnt) { settle_specials<XM>(F, Q, P, X, row, w, cnt, v4q, Rw, cw, m, theta, t1); };
    // The queue is filled in chunks of at most qcap <= QCAP entries, each holding
    // whole batches (a segment's lanes are settled together): chunk 0 in LDS,
    // chunks 1.. in this row's overflow area of the workspace, kQovfWave
    // entries per wave.  All are settled in phase F+X: phase S never
    // settles.  qch: current chunk,
    // qn: its entries, lane c of ccnt: the entries of an earlier chunk c.
    // (one block per workgroup: a workgroup samples one row at a time)
    uint32_t* const ovp = Q.qovf + (int64_t)wslot * kQovfRow + (int64_t)w * kQovfWave;
    const int qcap = (P.qcap > 0u && P.qcap < (uint32_t)QCAP) ? (int)P.qcap : QCAP;  // entries per chunk
    int qch = 0;
    uint32_t ccnt = 0;
    bool qovf = false;
    if (!F.fail) {
      // per-segment constants, lane k for this wave's segment k; segments
      // that are not PLAIN (or absent) get zero scales and an unreachable
      // tspec, so every bracket is MAGIC and no lane is special
      const bool plain_l = have && F.sflag[w + W * lane] == (uint8_t)PLAIN;
      const GridConst gc_l = grid_const(have ? (int)F.sj[w + W * lane] : 0, Rw, theta, fabsf(aw), t1, P.est_xe);
      const float sclo_l = plain_l ? gc_l.sc_lo : 0.0f;
      const float schi_l = plain_l ? gc_l.sc_hi : 0.0f;
      const uint32_t tsp_l = plain_l ? __float_as_uint(gc_l.tspec) : 0xffffffffu;
      // the same constants as an LDS table, read by the register batches
      // (an LDS read instead of three readlanes per segment), in LDS no
      // other wave writes before the walk ends
      float4* const ctab = &F.u.s.ctab[w][0];
      auto lds_q = [&](int k) {
        return to_v4(reinterpret_cast<const float4*>(&F.u.data[w][min(max(k - KV, 0), KL - 1)][0])[lane]);
      };
      // One batch: four segments k0 .. k0 + 3 (k0 a constant).  Per lane and
      // segment, the lower and upper bracket roundings of its four terms
      // (bit patterns of MAGIC + rounding); the lane is special when the
      // sums differ or a term reaches tspec (tsp).  Sums
      // wrap (the true values are far below 2^32); the segment sums keep the
      // offsets (4 MAGIC_BITS a lane, even), taken out in phase B.
      auto batch = [&](const int k0, const bool tab, const llz_f4v qa, const llz_f4v qb, const llz_f4v qc,
                       const llz_f4v qd) {
        uint32_t raw4[4];
        uint64_t spm[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          float sc_lo, sc_hi;
          uint32_t tsp;
          if (tab) {
            const float4 c = ctab[min(k0 + s, kWave - 1)];
            sc_lo = c.x;
            sc_hi = c.y;
            tsp = __float_as_uint(c.z);
          } else {
            const int kl = min(k0 + s, kWave - 1);
            sc_lo = readlane_f32(sclo_l, kl);
            sc_hi = readlane_f32(schi_l, kl);
            tsp = readlane_u32(tsp_l, kl);
          }
          const llz_f4v qv4 = s == 0 ? qa : s == 1 ? qb : s == 2 ? qc : qd;  // s is a constant here
          const uint32_t l0 = __float_as_uint(fmaf(qv4.x, sc_lo, MAGIC));
          const uint32_t l1 = __float_as_uint(fmaf(qv4.y, sc_lo, MAGIC));
          const uint32_t l2 = __float_as_uint(fmaf(qv4.z, sc_lo, MAGIC));
          const uint32_t l3 = __float_as_uint(fmaf(qv4.w, sc_lo, MAGIC));
          const uint32_t h0 = __float_as_uint(fmaf(qv4.x, sc_hi, MAGIC));
          const uint32_t h1 = __float_as_uint(fmaf(qv4.y, sc_hi, MAGIC));
          const uint32_t h2 = __float_as_uint(fmaf(qv4.z, sc_hi, MAGIC));
          const uint32_t h3 = __float_as_uint(fmaf(qv4.w, sc_hi, MAGIC));
          // bit patterns of non-negative floats order like their values: each
          // upper bracket is >= its lower one, so the sums agree exactly when
          // every pair does
          const uint32_t lsum = (l0 + l1) + (l2 + l3);
          const uint32_t hsum = (h0 + h1) + (h2 + h3);
          const uint32_t hmax = max(max(h0, h1), max(h2, h3));
          raw4[s] = lsum;
          // absent positions hold q = 0, so their brackets are MAGIC: never
          // special (tspec > MAGIC for PLAIN segments outside flood mode, and
          // theta is +inf in flood mode; the other segments have zero scales).
          // Two ballots straight from the compares
          spm[s] = __builtin_amdgcn_ballot_w64(hsum != lsum) | __builtin_amdgcn_ballot_w64(hmax >= tsp);
        }
        // segment sums in four parts, one per 16-lane row (lane 16 r + 12 + s
        // holds row r's part of segment k0 + s).  Every wave has room for 64
        // segments: absent ones store offsets only
        const uint32_t rsum = row_sums4(raw4[0], raw4[1], raw4[2], raw4[3]);
        if ((lane & 12) == 12) F.v.ssum4[w + W * (k0 + (lane & 3))][lane >> 4] = rsum;
        const int total = __popcll(spm[0]) + __popcll(spm[1]) + __popcll(spm[2]) + __popcll(spm[3]);
        if (total != 0) {
          if (total > qcap) {
            qovf = true;  // more uncertified lanes in four segments than a chunk holds
          } else {
            if (qn + total > qcap) {  // the batch starts the next chunk (chunks hold whole batches)
              ccnt = lane == qch ? qn : ccnt;
              ++qch;
              qn = 0;
              // chunk qch occupies entries [(qch - 1) qcap, qch qcap) of the wave's
              // kQovfWave; a wave that needs more fails the row (streaming normaliser)
              if (qch * qcap > kQovfWave || qch >= kWave) qovf = true;
            }
            uint32_t* const op = ovp + (qch - 1) * qcap;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
              if (spm[s] != 0ull) {
                // segment by segment, in lane order; a tie is decided by the
                // parity of the integer before it: per segment, that of the
                // lower bracket sum of the lanes below
                const uint64_t pm = __builtin_amdgcn_ballot_w64((raw4[s] & 1u) != 0u);
                const uint32_t par =
                    __builtin_amdgcn_mbcnt_hi((uint32_t)(pm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)pm, 0u));
                const int slot =
                    qn + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(spm[s] >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)spm[s], 0u));
                const uint32_t qp = (uint32_t)((w + W * (k0 + s)) * SEG + lane4) | (par << 31);
                if ((spm[s] >> lane) & 1ull) {
                  if (qch == 0)
                    F.qpos[w][slot] = qp;
                  else if (!qovf)
                    op[slot] = qp;
                }
                qn += __popcll(spm[s]);
              }
            }
          }
        }
      };
      // the batches holding LDS-resident segments first (k0 >= KV - 1), then
      // one barrier: every wave is past its LDS segments, so the EXACT slots
      // (which overlay them) can be re-read while the register batches run.
      // Every batch is unrolled with constant register indices (a runtime
      // switch over them costs a chain of branches per batch).
      static_assert((KV - 1) % 4 == 0, "batch KV - 1 is the first to hold LDS-resident segments");
      constexpr int kLdsBatches = (SPWMAX - (KV - 1) + 3) / 4;
#pragma unroll
      for (int b = 0; b < kLdsBatches; ++b) {
        const int k0 = (KV - 1) + 4 * b;
        if (k0 < nseg_w)
          batch(k0, false, k0 < KV ? to_v4(d[k0 < KV ? k0 : 0]) : lds_q(k0), lds_q(k0 + 1), lds_q(k0 + 2), lds_q(k0 + 3));
      }
      __syncthreads();
      LLZ_STAMP(row, 22);
      exact_loads<FASTLD>(F, xr, w, min(F.nslot, dcap), n);
      ctab[lane] = make_float4(sclo_l, schi_l, __uint_as_float(tsp_l), 0.0f);  // read by this wave only
#pragma unroll
      for (int b = 0; b < (KV - 1) / 4; ++b) {
        const int k0 = 4 * b;
        if (k0 < nseg_w) batch(k0, true, to_v4(d[k0]), to_v4(d[k0 + 1]), to_v4(d[k0 + 2]), to_v4(d[k0 + 3]));
      }
      ccnt = lane == qch ? qn : ccnt;  // the last chunk's entries
      if (qovf && lane == 0) atomicOr(&F.fail, 1u);
    }
    LLZ_STAMP(row, 3);

    // ---- phase F+X: this round's EXACT slots (re-read during phase S) and
    // the remaining specials, whose re-reads land while the slots are
    // evaluated
    if (!F.fail) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the EXACT slots' re-reads (and phase S's stores)
      LLZ_STAMP(row, 16);
      const int qn0 = (int)readlane_u32(ccnt, 0);
      reread(qn0);
      // this wave's EXACT slots (slot_step: slot 0 alone on wave 0, loaded by this wave),
      // while the re-reads land; slot 0, the row's first segment, needs no
      // tables: wave 0 sums it term by term
      for (int slot = w; slot < min(F.nslot, dcap); slot += slot_step(w)) {
        slot_terms(F, Q, P, X, row, slot, n, m, theta, t1);
        if (slot != 0) slot_tables(F, slot);
      }
      LLZ_STAMP(row, 17);
      if (w == 0) {
        // the row's first segment (slot 0) from 0, term by term as
        // sampler.zig:87 adds them: four chains of 64 terms, one term per
        // lane (absent positions hold 0).  The walk starts after it.
        const float* d0 = &F.u.x.dump[0][0];
        const float x0 = d0[lane], x1 = d0[kWave + lane], x2 = d0[2 * kWave + lane], x3 = d0[3 * kWave + lane];
        float s0 = readlane_f32(wave_chain_lanes<false>(0.0f, x0, kWave), kWave - 1);
        s0 = readlane_f32(wave_chain_lanes<false>(s0, x1, kWave), kWave - 1);
        s0 = readlane_f32(wave_chain_lanes<false>(s0, x2, kWave), kWave - 1);
        s0 = readlane_f32(wave_chain_lanes<false>(s0, x3, kWave), kWave - 1);
        if (lane == 0) {
          F.s_run = s0;
          F.next_e = 1;
        }
      }
      LLZ_STAMP(row, 18);
      settle(qn0);
      LLZ_STAMP(row, 19);
      // the chunks past the LDS queue (rare)
      for (int c = 1; c <= qch; ++c) {
        const int cn = (int)readlane_u32(ccnt, c);
        for (int i = lane; i < cn; i += kWave) F.qpos[w][i] = ovp[(c - 1) * qcap + i];
        reread(cn);
        settle(cn);
      }
    }
    __syncthreads();
    LLZ_STAMP(row, 4);

    // ---- phase B: the walk's entries, built in parallel (wave c takes
    // segments 64c .. 64c + 63, one per lane): a run of PLAIN segments on one
    // binade becomes one entry with its integer sum; PLAIN_TIE and EXACT
    // segments are one entry each
    constexpr uint32_t E_RUN = 0, E_TIE = 1, E_EXACT = 2;
    if (!F.fail) {
      const int g = kWave * w + lane;
      const bool in = g < G;
      const uint32_t fl = in ? F.sflag[g] : (uint32_t)EXACT_PRED;
      const int jj = in ? F.sj[g] : 0;
      uint32_t sm = 0u;
      if (in) {
        const uint4 p4 = *reinterpret_cast<const uint4*>(&F.v.ssum4[g][0]);
        sm = min(p4.x + p4.y + p4.z + p4.w - (uint32_t)(kWave * 4) * MAGIC_BITS, kSat);
      }
      const bool plain = in && fl == PLAIN;
      const uint32_t key = plain ? (0x10000u | (uint32_t)(jj & 0xffff)) : 0u;
      const bool head = in && !(plain && wave_shift_up1(key) == key);
      const uint64_t heads = bal64(head);
      // a run's sum up to this lane: the inclusive prefix minus the exclusive
      // prefix at the run's head (prefixes never decrease, so a max-scan of the
      // heads' exclusive prefixes yields the latest head's); <= 64 * 2^25: no wrap
      const uint32_t v = plain ? sm : 0u;
      const uint32_t pin = wave_incl_scan_op(v, 0u, [](uint32_t a, uint32_t b) { return a + b; });
      const uint32_t hb = wave_incl_scan_op(head ? pin - v : 0u, 0u, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
      const bool tail = plain && (lane == kWave - 1 || g + 1 >= G || ((heads >> (lane + 1)) & 1ull) != 0ull);
      if (lane == 0) F.wnex[w] = __popcll(heads);
      __syncthreads();
      int off = 0, ne = 0;
      for (int i = 0; i < W; ++i) {
        if (i < w) off += F.wnex[i];
        ne += F.wnex[i];
      }
      if (head) {
        const uint32_t type = plain ? E_RUN : (fl == PLAIN_TIE ? E_TIE : E_EXACT);
        const uint32_t tb = fl == PLAIN_TIE ? (uint32_t)F.sbump[g] : 0u;
        F.u.x.ent_a[off + __popcll(heads & lt_mask)] =
            type | ((uint32_t)g << 2) | ((uint32_t)(jj + 128) << 16) | (tb << 24);
        // PLAIN_TIE: its integer sum; EXACT: its round-0 slot and grid count
    if (!plain)
      F.u.x.ent_b[off + __popcll(heads & lt_mask)] =
          fl == PLAIN_TIE ? sm : (uint32_t)(uint8_t)F.sdump[g] | ((uint32_t)F.sng[g] << 8);
      }
      if (tail) F.u.x.ent_b[off + __popcll(heads & (lt_mask | (1ull << lane))) - 1] = pin - hb;
      if (t == 0) F.ne = ne;
    }
    __syncthreads();
    LLZ_STAMP(row, 5);

    // waves 1.. read the candidate list while wave 0 walks, one entry per
    // thread from thread 64 on (entries a later round collects are read at
    // the hand-over)
    cand_n0 = F.ncand;
    if (w > 0 && t - kWave < (int)min(cand_n0, (uint32_t)kCandCap))
      cand_pre = Q.cand[(int64_t)row * kCandCap + (t - kWave)];
    // ---- phase C: the walk over the entries in index order (wave 0); EXACT
    // segments beyond the slots in further rounds
    LLZ_STAMP(row, 20);
    for (int round = 0; !F.fail; ++round) {
      if (round > 0) {
        if (t == 0) F.diag |= kPathWalkRounds;
        if (w == 0) {  // slots for the EXACT segments from the stopping entry's on, in order
          const int g_from = (int)((F.u.x.ent_a[F.next_e] >> 2) & 1023u);
          int cnt = 0;
          for (int b = g_from; b < G; b += kWave) {
            const int g = b + lane;
            const bool ex = g < G && (F.sflag[g] == EXACT_PRED || F.sflag[g] == EXACT_DONE);
            const uint64_t mk = bal64(ex);
            const int slot = cnt + __popcll(mk & lt_mask);
            if (ex) {
              F.sdump[g] = (int8_t)(slot < dcap ? slot : -1);
              if (slot < dcap) F.slotseg[slot] = (int16_t)g;
            }
            cnt += __popcll(mk);
          }
          if (lane == 0) F.nslot = min(cnt, dcap);
        }
        __syncthreads();
        const int nslot = F.nslot;
        exact_loads<FASTLD>(F, xr, w, nslot, n);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        exact_segments(F, Q, P, X, row, w, nslot, n, m, theta, t1);
        __syncthreads();
      }
      if (w == 0) {
        // the running sum as N on grid jc, in scalar registers
        const Grid g0 = grid_of(uni_f(F.s_run));
        uint32_t N = g0.N;
        int jc = g0.j;
        int e = F.next_e;
        const int ne = F.ne;
        bool fail = false, more = false;
        // windows of 64 entries, one per lane.  What does not depend on the
        // running sum is computed for every lane at once: for an EXACT lane x,
        // its slot, grids and the stretch of runs (and PLAIN_TIE segments)
        // between the previous EXACT entry and x: the stretch's sum (a
        // difference of a prefix sum), its grid, and whether it can be added
        // in one step (no tie, one grid).  The walk then takes the EXACT
        // entries in order, reading ahead the next one's slot data while it
        // resolves this one.
        constexpr uint32_t XI_CLEAN = 1u << 27, XI_EMPTY = 1u << 28;
        for (int held = e & ~(kWave - 1); held < ne && !fail && !more; held += kWave) {
          const bool ok = held + lane < ne;
          const uint32_t ea = ok ? F.u.x.ent_a[held + lane] : 0u;
          const uint32_t eb = ok ? F.u.x.ent_b[held + lane] : 0u;
          const int ej = (int)((ea >> 16) & 0xffu) - 128;
          const bool isx = ok && (ea & 3u) == E_EXACT;
          const uint64_t exm = bal64(isx);
          const uint64_t tim = bal64(ok && (ea & 3u) == E_TIE);
          // <= 64 * 2^25: no wrap
          const uint32_t psum =
              wave_incl_scan_op(ok && !isx ? eb : 0u, 0u, [](uint32_t a, uint32_t b) { return a + b; });
          const int wend = min(ne - held, kWave);
          const int ejp = (int)wave_shift_up1((uint32_t)ej);  // the entry before's grid
          // entries whose grid differs from the entry before (neither EXACT)
          const uint64_t chg = bal64(ok && !isx && lane > 0 && ej != ejp) & ~(exm << 1);
          // the stretch ending at this lane: entries pv + 1 .. lane - 1
          const uint64_t xb = exm & lt_mask;
          const int pv = xb != 0ull ? 63 - __builtin_clzll(xb) : -1;
          const uint32_t psum_pv = (uint32_t)__builtin_amdgcn_ds_bpermute(max(pv, 0) << 2, (int)psum);
          const uint32_t sts = psum - (pv >= 0 ? psum_pv : 0u);  // an EXACT lane adds 0 to psum
          const uint64_t upto = pv >= 0 ? (~0ull >> (63 - pv)) : 0ull;  // lanes 0 .. pv
          const uint64_t span = lt_mask & ~upto;
          const bool clean = (tim & span) == 0ull && (chg & span & ~(upto << 1 | 1ull)) == 0ull;
          int slot_l = (int)(int8_t)(eb & 0xffu);
          if (round > 0 && isx) slot_l = F.sdump[(ea >> 2) & 1023u];  // slots were reassigned
          const uint32_t xi = (uint32_t)(slot_l & 0xff) | ((uint32_t)(ej + 128) << 8) | ((uint32_t)(ejp + 128) << 16) |
                              (((eb >> 8) & 7u) << 24) | (clean ? XI_CLEAN : 0u) | (pv == lane - 1 ? XI_EMPTY : 0u);
          auto xslot_of = [](uint32_t a) { return (int)(int8_t)(a & 0xffu); };
          int i = e - held;
          int last = i - 1;  // the last entry consumed
          // the next EXACT entry's data is read without branches (an absent
          // one reads lane 0 and slot 0, unused)
          uint64_t rem = exm & (~0ull << i);
          int x = rem != 0ull ? __ffsll((long long)rem) - 1 : -1;
          uint32_t a = uni_u(readlane_u32(xi, x & (kWave - 1)));
          SlotAhead X = slot_ahead(F, max(xslot_of(a), 0));
          while (x >= 0) {
            rem &= rem - 1ull;
            const int x2 = rem != 0ull ? __ffsll((long long)rem) - 1 : -1;
            const uint32_t a2 = uni_u(readlane_u32(xi, x2 & (kWave - 1)));
            const SlotAhead X2 = slot_ahead(F, max(xslot_of(a2), 0));
            // the stretch before x on grid jc (added already when x resumes a
            // round): terms are >= 0, so it stays in the binade exactly when
            // its total does.  The common case (one step, or nothing) without
            // a branch
            const bool skip = (a & XI_EMPTY) != 0u || (x == i && round > 0);
            if (__builtin_expect(skip || (a & XI_CLEAN) != 0u, 1)) {
              N += skip ? 0u : readlane_u32(sts, x);
              const bool bad = !skip && (int)((a >> 16) & 0xffu) - 128 != jc;
              if (__builtin_expect(bad || N >= kGridTop, 0)) {
                fail = true;  // the running sum is not in the predicted binade, or leaves it
                break;
              }
            } else {
              // a PLAIN_TIE segment adds the units its ties take for the
              // parity of the integer it starts at: one entry at a time
              bool bad = false;
              for (int r = last + 1; r < x; ++r) {
                const uint32_t ra = readlane_u32(ea, r), rb = readlane_u32(eb, r);
                const uint32_t tu = ra >> 24;
                const uint32_t bump = (ra & 3u) == E_TIE ? ((N & 1u) ? (tu >> 4) : (tu & 15u)) : 0u;
                bad = bad || (int)((ra >> 16) & 0xffu) - 128 != jc || N >= kGridTop;
                N += rb + bump;
              }
              if (bad || N >= kGridTop) {
                fail = true;
                break;
              }
            }
            if (__builtin_expect(xslot_of(a) < 0, 0)) {
              more = true;  // EXACT segments past this round's slots
              last = x - 1;
              break;
            }
            resolve_ahead(N, jc, xslot_of(a), (int)((a >> 8) & 0xffu) - 128, (int)((a >> 24) & 7u), X, F);
            last = x;
            x = x2;
            a = a2;
            X = X2;
          }
          if (!fail && !more && last < wend - 1) {
            // the window's last stretch: entries last + 1 .. wend - 1
            const uint64_t tspan = (wend >= kWave ? ~0ull : ((1ull << wend) - 1ull)) & (~0ull << (last + 1));
            const uint64_t gspan = tspan & ~(1ull << (last + 1));
            bool bad;
            if ((tim & tspan) == 0ull && (chg & gspan) == 0ull) {
              N += readlane_u32(psum, wend - 1) - (last >= 0 ? readlane_u32(psum, last) : 0u);
              bad = (int)readlane_u32((uint32_t)ej, last + 1) != jc;
            } else {
              bad = false;
              for (int r = last + 1; r < wend; ++r) {
                const uint32_t ra = readlane_u32(ea, r), rb = readlane_u32(eb, r);
                const uint32_t tu = ra >> 24;
                const uint32_t bump = (ra & 3u) == E_TIE ? ((N & 1u) ? (tu >> 4) : (tu & 15u)) : 0u;
                bad = bad || (int)((ra >> 16) & 0xffu) - 128 != jc || N >= kGridTop;
                N += rb + bump;
              }
            }
            if (bad || N >= kGridTop) fail = true;
            last = wend - 1;
          }
          e = held + last + 1;
        }
        LLZ_STAMP(row, 21);
        if (lane == 0) {
          F.s_run = __uint_as_float(grid_bits(N, jc));
          F.next_e = e;
          if (fail) F.fail = 1u;
          F.done = (!fail && !more) ? 1 : 0;
        }
      }
      __syncthreads();
      if (F.done) break;
    }

    // ---- hand-over to the selection stage
    LLZ_STAMP(row, 6);
    certified = F.fail == 0u;
    S = F.s_run;
    cc = flood ? (uint32_t)kCandCap + 1u : F.ncand;
    pre_ok = !flood && cc <= (uint32_t)(NT - kWave);
  }

  // ---- the selection stage, on the same workgroup and shared memory.  It
  // writes only the first sizeof(SampleShared) bytes, inside F.u, which
  // nothing reads after the walk's last barrier (the fields read since, the
  // walk's results, lie past F.u): no barrier here
  static_assert(sizeof(SampleShared) <= sizeof(F.u), "the selection's memory must lie inside F.u");
  select_row(P, Q, U.select, m, certified ? S : 0.0f, certified ? cc : 0u, !certified, u_row, certified && pre_ok,
             cand_pre, cand_n0, X, O, XF ? &pen_sh : nullptr, kernel_args_ptr(), row);
  LLZ_STAMP(row, 15);
  // the walk's diagnostics join the status thread 0 wrote (F.diag lies past
  // the selection's memory)
  if (t == 0 && Q.status) {
    const uint32_t d = F.diag;
    if (d != 0u) Q.status[row] |= d;
  }
}

// One row per workgroup: launches whose rows fit the CUs at once.
template <bool FASTLD, int XM, bool EXT>
__global__ __launch_bounds__(NT) void k_stats(KArgs A) {
  __shared__ StatsShared U;
  __shared__ PenShared pen_sh;  // kXfPen: the row's penalised positions
  stats_row<FASTLD, XM, EXT>(A, (int)blockIdx.x, U, pen_sh, (int)blockIdx.x);
}

// More rows than CUs: one workgroup per CU (all resident), each taking rows
// [0, grid) one each and then claiming the next unclaimed row until none is
// left, so rows of unequal cost spread over every CU.  (Launched one row per
// workgroup instead, the hardware hands workgroups to the XCDs in turn, so a
// batch whose cost alternates from row to row loads half of the XCDs only.)
template <bool FASTLD, int XM, bool EXT>
__global__ __launch_bounds__(NT) void k_stats_rows(KArgs A) {
  __shared__ StatsShared U;
  __shared__ PenShared pen_sh;
  __shared__ int next_row;
  for (int row = (int)blockIdx.x;;) {
    // the arguments through a pointer the compiler cannot see through, so
    // that each row loads them where it uses them instead of holding them in
    // registers across rows
    const __attribute__((address_space(4))) KArgs* Ap =
        (const __attribute__((address_space(4))) KArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(Ap));
    stats_row<FASTLD, XM, EXT>(*(const KArgs*)Ap, row, U, pen_sh, (int)blockIdx.x);
    if (threadIdx.x == 0) next_row = claim_row(A.Q.claim, A.P.epoch, A.P.grid);
    __syncthreads();  // also: every wave is done with this row's shared memory
    row = next_row;
    if (row >= A.P.rows) return;
  }
}

// Split rows (token-only calls of few rows, plain 16-byte aligned rows):
// workgroup b reads chunk b % split_s of row b / split_s (NV float4 per
// thread); a workgroup that sees the row's chunks published merges it, and
// the one that takes an uncertified row finishes it with the single-row
// path of k_stats (its overflow block: the row's, rows <= kSplitRows <
// kMaxGrid).
union SplitLds {
  SplitShared split;
  StatsShared stats;
};
template <int NV, int XM>
__global__ __launch_bounds__(NT) void k_split(KArgs A) {
  __shared__ SplitLds U;
  __shared__ PenShared pen_sh;  // the single-row path's penalised positions (kXfPen)
  const int ns = A.P.split_s;
  const int row = (int)blockIdx.x / ns, c = (int)blockIdx.x - row * ns;
  if (!split_chunk<NV, XM != kXmNone>(A, row, c, U.split)) return;
  if (split_merge(A, row, U.split)) return;
  if (!split_take(A, row, U.split)) return;  // (its barrier: every wave is done with the merge's shared memory)
  stats_row<true, XM>(A, row, U.stats, pen_sh, row);
}

}  // namespace

// One launch per call: every row's statistics, then its selection.
hipError_t launch_sample(const RowParams& P, const RowPtrs& Q, hipEvent_t ev_begin, hipEvent_t ev_end,
                         hipStream_t st) {
  if (ev_begin && hipEventRecord(ev_begin, st) != hipSuccess) return hipErrorUnknown;
  const bool fastld = (P.flags & kFlagVecSrc) != 0 && (P.n % 4) == 0;
  // the transform mode: soft-capping (the chain's input) takes the
  // estimating single pass, the scale and the penalty alone the exact one
  const int xm = (P.xf_src & kXfCap) ? kXmCap : ((P.xf_src | P.xf_orig) != 0u ? kXmLight : kXmNone);
  const KArgs A{P, Q};
  // more rows than workgroups: the grid's workgroups claim rows (the
  // special-queue overflow area has one block per workgroup of the grid)
  const bool claim = P.grid < P.rows;
  // transformed rows split with chunks of at most 2 float4 per thread (each
  // logit's exact post-processing is then a few per thread)
  const bool split = P.split_s >= 2 && fastld && P.rows <= kSplitRows && (xm == kXmNone || P.split_nv <= 2);
  // token-only calls with typical-p (not soft-capped) take the instantiation
  // that carries typical-p's decisions and the list's second collection
  // round; the others keep the shorter code
  const bool ext = (P.flags & kFlagTokenOnly) != 0u && P.typical_p > 0.0f && P.typical_p < 1.0f && xm != kXmCap;
  const dim3 grid(split ? P.rows * P.split_s : (claim ? P.grid : P.rows)), block(NT);
  void (*kern)(KArgs) = nullptr;
  if (split) {
    if (xm == kXmNone) {
      switch (P.split_nv) {
        case 1: kern = k_split<1, kXmNone>; break;
        case 2: kern = k_split<2, kXmNone>; break;
        case 4: kern = k_split<4, kXmNone>; break;
        case 8: kern = k_split<8, kXmNone>; break;
        default: return hipErrorInvalidValue;
      }
    } else if (xm == kXmLight) {
      kern = P.split_nv == 1 ? k_split<1, kXmLight> : k_split<2, kXmLight>;
    } else {
      kern = P.split_nv == 1 ? k_split<1, kXmCap> : k_split<2, kXmCap>;
    }
  } else if (claim) {
    if (ext)
      kern = fastld ? (xm == kXmNone ? k_stats_rows<true, kXmNone, true> : k_stats_rows<true, kXmLight, true>)
                    : (xm == kXmNone ? k_stats_rows<false, kXmNone, true> : k_stats_rows<false, kXmLight, true>);
    else if (fastld)
      kern = xm == kXmNone ? k_stats_rows<true, kXmNone, false> : xm == kXmLight ? k_stats_rows<true, kXmLight, false>
                                                                                 : k_stats_rows<true, kXmCap, false>;
    else
      kern = xm == kXmNone ? k_stats_rows<false, kXmNone, false> : xm == kXmLight ? k_stats_rows<false, kXmLight, false>
                                                                                  : k_stats_rows<false, kXmCap, false>;
  } else {
    if (ext)
      kern = fastld ? (xm == kXmNone ? k_stats<true, kXmNone, true> : k_stats<true, kXmLight, true>)
                    : (xm == kXmNone ? k_stats<false, kXmNone, true> : k_stats<false, kXmLight, true>);
    else if (fastld)
      kern = xm == kXmNone ? k_stats<true, kXmNone, false> : xm == kXmLight ? k_stats<true, kXmLight, false>
                                                                            : k_stats<true, kXmCap, false>;
    else
      kern = xm == kXmNone ? k_stats<false, kXmNone, false> : xm == kXmLight ? k_stats<false, kXmLight, false>
                                                                             : k_stats<false, kXmCap, false>;
  }
  void* args[] = {const_cast<KArgs*>(&A)};
  if (hipLaunchKernel((const void*)kern, grid, block, args, 0, st) != hipSuccess) return hipErrorLaunchFailure;
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (ev_end && hipEventRecord(ev_end, st) != hipSuccess) return hipErrorUnknown;
  return hipSuccess;
}

}  // namespace llz

#ifdef LLZ_PHASE_STAMPS
// Measurement builds: the phase timestamps of rows 0 .. rows - 1 (kStampSlots
// per row, 0 where a row did not reach the boundary) into dst.
extern "C" int llz_debug_phase_stamps(unsigned long long* dst, int rows, int clear) {
  if (rows <= 0 || rows > llz::kStampRows || !dst) return -1;
  const size_t bytes = (size_t)rows * llz::kStampSlots * sizeof(unsigned long long);
  if (clear) {
    static unsigned long long zeros[llz::kStampRows * llz::kStampSlots];
    return hipMemcpyToSymbol(HIP_SYMBOL(llz::llz_phase_stamps), zeros, sizeof(zeros)) == hipSuccess ? 0 : -3;
  }
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(llz::llz_phase_stamps), bytes) == hipSuccess ? 0 : -3;
}
#endif
