// llz_stats.hip -- k_stats: single-pass row statistics for the sampling chain
// (sampler.zig:80-88): the row maximum, the exact sequential f32 normaliser
// and the candidate list, with one HBM read per logit.  The method and its
// error bound are described in llz_fast.h.  Rows it cannot certify are
// flagged in row_state[3]; k_select then runs the streaming normaliser on
// them.
#include <hip/hip_runtime.h>

#include "llz_exact.h"
#include "llz_fast.h"
#include "llz_internal.h"
#include "llz_math.h"
#include "llz_norm.h"
#include "llz_wg.h"

namespace llz {
namespace {

using namespace fastp;
constexpr float kInfS = __builtin_inff();


// d[k] for a wave-uniform runtime k: every case reads a fixed register.
__device__ __forceinline__ float4 pick(const float4 (&d)[KV], int k) {
  float4 r = d[0];
  switch (k) {
#define LLZ_PICK(i) \
  case i:           \
    r = d[i];       \
    break;
    LLZ_PICK(0) LLZ_PICK(1) LLZ_PICK(2) LLZ_PICK(3) LLZ_PICK(4) LLZ_PICK(5) LLZ_PICK(6) LLZ_PICK(7)
    LLZ_PICK(8) LLZ_PICK(9) LLZ_PICK(10) LLZ_PICK(11) LLZ_PICK(12) LLZ_PICK(13) LLZ_PICK(14) LLZ_PICK(15)
    LLZ_PICK(16) LLZ_PICK(17) LLZ_PICK(18) LLZ_PICK(19) LLZ_PICK(20) LLZ_PICK(21) LLZ_PICK(22) LLZ_PICK(23)
    LLZ_PICK(24) LLZ_PICK(25) LLZ_PICK(26) LLZ_PICK(27) LLZ_PICK(28) LLZ_PICK(29) LLZ_PICK(30) LLZ_PICK(31)
    LLZ_PICK(32) LLZ_PICK(33) LLZ_PICK(34) LLZ_PICK(35) LLZ_PICK(36) LLZ_PICK(37) LLZ_PICK(38) LLZ_PICK(39)
    LLZ_PICK(40) LLZ_PICK(41) LLZ_PICK(42) LLZ_PICK(43) LLZ_PICK(44)
#undef LLZ_PICK
  }
  return r;
}
static_assert(KV == 45, "pick() covers 45 register segments");

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
__device__ __forceinline__ uint32_t nan4(float4 v) {
  return (uint32_t)((v.x != v.x) | (v.y != v.y) | (v.z != v.z) | (v.w != v.w));
}

__device__ __forceinline__ void push_cand(FastShared& F, const RowPtrs& Q, int row, float e, uint32_t id) {
  const uint32_t slot = atomicAdd(&F.ncand, 1u);
  if (slot < (uint32_t)kCandCap) Q.cand[(int64_t)row * kCandCap + slot] = ((uint64_t)__float_as_uint(e) << 32) | id;
}

// Owner wave: its EXACT segments that hold a dump slot, at or after g_from,
// as a bit mask over the wave's segments (bit k: segment seg0 + k).
__device__ __forceinline__ uint64_t exact_mask(const FastShared& F, int seg0, int nseg_w, int g_from) {
  const int lane = lane_id();
  const int seg = seg0 + lane;
  const bool ex = lane < nseg_w && seg >= g_from && F.sflag[seg] != PLAIN && F.sdump[seg] >= 0;
  return __ballot(ex);
}

// Owner wave: exact terms of the EXACT segments in `mask` (their loads were
// issued and waited for by the caller), their candidates, and the per-lane
// prefix tables of the roundings on grids sj and sj+1.
__device__ __forceinline__ void exact_segments(FastShared& F, const RowPtrs& Q, const RowParams& P, int row, int seg0,
                                               uint64_t mask, int n, float m, float theta, bool t1) {
  const int lane = lane_id();
  while (mask != 0ull) {
    const int k = __ffsll((long long)mask) - 1;
    mask &= mask - 1ull;
    const int seg = seg0 + k;
    const int slot = F.sdump[seg];
    const bool pred = F.sflag[seg] == EXACT_PRED;
    float4* p = reinterpret_cast<float4*>(&F.u.x.dump[slot][lane * 4]);
    const float4 v = *p;
    const float vs[4] = {v.x, v.y, v.z, v.w};
    float es[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int pos = seg * SEG + lane * 4 + c;
      es[c] = pos < n ? exact_term(vs[c], m, P.temperature, t1) : 0.0f;
      if (pred && pos < n && es[c] >= theta) push_cand(F, Q, row, es[c], (uint32_t)pos);
    }
    *p = make_float4(es[0], es[1], es[2], es[3]);
    if (pred && lane == 0) F.sflag[seg] = EXACT_DONE;  // a later round must not collect them again
    const int J0 = F.sj[seg];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      uint32_t sum = 0;
      bool tie_any = false;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        bool tie;
        sum = sat_add(sum, grid_round(es[c], J0 + kk, tie), kSat);
        tie_any = tie_any || tie;
      }
      F.u.x.pref[slot][kk][lane] = wave_incl_scan_sat(sum, kSat);
      const uint64_t tm = __ballot(tie_any);
      if (lane == 0) F.u.x.tmask[slot][kk] = tm;
    }
  }
}

// Owner wave: issue the re-reads of the EXACT segments in `mask` into their slots.
template <bool FASTLD>
__device__ __forceinline__ void exact_loads(FastShared& F, const float* xr, int seg0, uint64_t mask, int n) {
  while (mask != 0ull) {
    const int k = __ffsll((long long)mask) - 1;
    mask &= mask - 1ull;
    const int seg = seg0 + k;
    seg_to_lds(xr, seg, n, FASTLD, &F.u.x.dump[F.sdump[seg]][0]);
  }
}

// Combine wave: the exact sequential sum across EXACT segment `slot` from
// the running value s, using the prefix tables (grids J0, J0+1) between
// events and replaying the lane that holds an event term by term.
__device__ __forceinline__ float resolve_exact(float s, int slot, int J0, const FastShared& F) {
  const int lane = lane_id();
  const float4 e4 = *reinterpret_cast<const float4*>(&F.u.x.dump[slot][lane * 4]);
  int p = 0;  // first lane not consumed
  for (int guard = 0; guard <= kWave && p < kWave; ++guard) {
    const Grid gr = grid_of(s);
    const int k = gr.j - J0;
    if (k < 0 || k > 1) {
      // outside the tabulated grids: the generic exact accumulation
      const float x[4] = {lane >= p ? e4.x : -0.0f, lane >= p ? e4.y : -0.0f, lane >= p ? e4.z : -0.0f,
                          lane >= p ? e4.w : -0.0f};
      return wave_accumulate<4>(s, x);
    }
    const uint32_t pv = F.u.x.pref[slot][k][lane];
    const uint32_t base = p > 0 ? F.u.x.pref[slot][k][p - 1] : 0u;
    const uint64_t live = p == 0 ? ~0ull : (~0ull << p);
    const bool cr = lane >= p && (pv >= kSat || gr.N + (pv - base) >= kGridTop);
    const uint64_t ev = (__ballot(cr) | F.u.x.tmask[slot][k]) & live;
    if (ev == 0ull) return grid_value(gr.N + (F.u.x.pref[slot][k][kWave - 1] - base), gr.j);
    const int E = __ffsll((long long)ev) - 1;
    if (E > p) s = grid_value(gr.N + (F.u.x.pref[slot][k][E - 1] - base), gr.j);
    // the lane holding the event, term by term (sampler.zig:87)
    s = s + readlane_f32(e4.x, E);
    s = s + readlane_f32(e4.y, E);
    s = s + readlane_f32(e4.z, E);
    s = s + readlane_f32(e4.w, E);
    p = E + 1;
  }
  return s;
}

// FASTLD: 16-byte aligned rows with n % 4 == 0 (one float4 per lane per
// segment through buffer loads); otherwise element loads.
template <bool FASTLD>
__global__ __launch_bounds__(NT) void k_stats(RowParams P, RowPtrs Q) {
  __shared__ FastShared F;
  const int row = blockIdx.x;
  const int t = (int)threadIdx.x, lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(wave_id());  // wave-uniform: scalar registers
  const int n = P.n;
  const bool t1 = (P.flags & kFlagTIsOne) != 0;
  const float* xr = Q.src + (int64_t)row * P.src_stride;
  const float l2e_t = P.l2e_t;
  const int G = (n + SEG - 1) / SEG;
  const int SPW = (G + W - 1) / W;
  const bool fits = SPW <= SPWMAX && P.cand_theta > 0.0f && fabsf(l2e_t) <= 0x1p40f;
  const int seg0 = w * SPW;
  const int nseg_w = fits ? max(0, min(SPW, G - seg0)) : 0;
  const int base_w = seg0 * SEG + lane * 4;
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
  float* rs_out = Q.row_state + (int64_t)row * 4;

  // ---- phase L: every load in flight, then per segment as it lands: running
  // maximum, the estimate q (stored over v) and the segment sum of q
  // Every load is issued unconditionally and fully unrolled (a guarded load
  // is sunk into its guard and waited for on its own): segments this wave
  // does not own read a valid address and are masked to -inf.
  float4 d[KV];
  if constexpr (FASTLD) {
    // LDS-resident segments straight to LDS (full ones; the partial last
    // segment and absent ones read the row start and are redone or unused)
#pragma unroll
    for (int k = KV; k < SPWMAX; ++k) {
      int kk = k;
      asm volatile("" : "+s"(kk));
      const bool full = kk < nseg_w && (seg0 + kk + 1) * SEG <= n;
      dma16(xr + (full ? base_w + kk * SEG : lane * 4),
            (uint32_t)__builtin_amdgcn_readfirstlane((int)(uintptr_t)&F.u.data[w][k - KV][0]));
    }
    // register segments: one shared lane offset, the segment offset in an
    // SGPR; reads past the row return 0
    const llz_i4v rs = row_rsrc(xr, (uint32_t)n * 4u);
    const int soff = __builtin_amdgcn_readfirstlane(seg0 * SEG * 4);
#pragma unroll
    for (int k = 0; k < KV; ++k) {
      d[k] = buf_ld4(rs, lane * 16, soff + k * SEG * 4);
      __builtin_amdgcn_sched_barrier(0);  // keep the issue order: segment k lands k-th
    }
  } else {
#pragma unroll
    for (int k = 0; k < KV; ++k) d[k] = ld1x4(xr, base_w + k * SEG, k < nseg_w ? n : 0);
    for (int k = KV; k < nseg_w; ++k) seg_to_lds(xr, seg0 + k, n, false, &F.u.data[w][k - KV][0]);
  }
  __builtin_amdgcn_sched_barrier(0);  // every load in flight before any use

  float mx = -kInfS, cw = 0.0f;
  uint32_t nanf = 0;
  // bounds as (lane offset, VGPR) < (scalar limit of the segment); the
  // limits are recomputed in place (an empty asm keeps the compiler from
  // hoisting 45 of them into live registers)
  const int lane4 = lane * 4;
  const int lim_w = min(n - seg0 * SEG, nseg_w * SEG);  // this wave's positions < lim_w
  auto seg_lim = [&](int k) {
    int l = lim_w - k * SEG;
    asm volatile("" : "+s"(l));
    return l;
  };
  {
    const bool ok0 = lane4 < seg_lim(0);
    float mr = wave_max_f32(ok0 ? max4(d[0]) : -kInfS);
    if (!(fabsf(mr) <= 3.0e38f)) mr = 0.0f;  // any finite reference: |m - mr| is checked below
    cw = mr * l2e_t;
  }
  // segment sums are kept one per lane (lane k: segment k) and stored after
  // the loop: an LDS access here would wait for the LDS-bound loads
  float my_a = 0.0f;
#pragma unroll
  for (int k = 0; k < KV; ++k) {
    const float4 v = d[k];
    const bool ok = lane4 < seg_lim(k);  // this wave's and inside the row
    mx = fmaxf(mx, ok ? max4(v) : -kInfS);
    float4 q = q_of(v, l2e_t, cw);  // a NaN logit makes its segment sum NaN
    q.x = ok ? q.x : 0.0f;
    q.y = ok ? q.y : 0.0f;
    q.z = ok ? q.z : 0.0f;
    q.w = ok ? q.w : 0.0f;
    // materialise q here, while the loads land (not sunk into phase S)
    asm volatile("" : "+v"(q.x), "+v"(q.y), "+v"(q.z), "+v"(q.w));
    d[k] = q;
    const float a = wave_sum_f32((q.x + q.y) + (q.z + q.w));
    my_a = lane == k ? a : my_a;
    __builtin_amdgcn_sched_barrier(0);  // one segment at a time: bounded live ranges
  }
  if (lane < min(nseg_w, KV)) F.aseg[seg0 + lane] = my_a;
  nanf = (lane < min(nseg_w, KV) && my_a != my_a) ? 1u : 0u;
  if (nseg_w > KV) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (FASTLD && (seg0 + nseg_w) * SEG > n) {  // the row's partial last segment
      const int k = nseg_w - 1;
      *reinterpret_cast<float4*>(&F.u.data[w][k - KV][lane * 4]) = ld4(xr, base_w + k * SEG, n);
    }
  }
  for (int k = KV; k < nseg_w; ++k) {
    float4* p = reinterpret_cast<float4*>(&F.u.data[w][k - KV][lane * 4]);
    const float4 v = *p;
    mx = fmaxf(mx, max4(v));
    const float4 q = q_of(v, l2e_t, cw);
    *p = q;
    const float a = wave_sum_f32((q.x + q.y) + (q.z + q.w));
    if (lane == 0) F.aseg[seg0 + k] = a;
    nanf |= a != a ? 1u : 0u;
  }
  if (!fits) {  // rows the fast path does not take: maximum and NaN scan only
    for (int i = t; i < n; i += NT) {
      const float v = xr[i];
      mx = fmaxf(mx, v);
      nanf |= (uint32_t)(v != v);
    }
  }
  mx = wave_max_f32(mx);
  const bool wnan = __ballot(nanf != 0u) != 0ull;
  if (lane == 0) {
    F.mw[w] = mx;
    F.cw[w] = cw;
    F.nanw[w] = wnan ? 1u : 0u;
  }
  if (t == 0) {
    F.fail = fits ? 0u : 1u;
    F.flood = 0;
    F.ncand = 0;
    F.next_g = 0;
    F.s_run = 0.0f;
    F.done = 0;
  }
  __syncthreads();

  // ---- phase M: row maximum, scale factors, binade prediction, first slots
  float m = -kInfS;
  bool nanrow = false;
#pragma unroll
  for (int i = 0; i < W; ++i) {
    m = fmaxf(m, F.mw[i]);
    nanrow = nanrow || F.nanw[i] != 0u;
  }
  if (nanrow || !(fabsf(m) <= 3.0e38f)) {
    // a NaN logit or an infinite maximum makes the reference's sum NaN
    if (t == 0) {
      rs_out[0] = m;
      rs_out[1] = __builtin_nanf("");
      rs_out[2] = __uint_as_float(0u);
      rs_out[3] = 0.0f;
    }
    return;
  }
  const float aw = fmaf(m, -l2e_t, cw);
  const float Rw = __builtin_amdgcn_exp2f(aw);  // q * Rw ~ e = exp((v - m) / T)
  // each wave predicts its own segments (one per lane); wave totals give the carries
  const bool have = lane < nseg_w;
  {
    const float a_l = have ? F.aseg[seg0 + lane] * Rw : 0.0f;
    const float sc = wave_incl_scan_f32(a_l);
    const float tot = __uint_as_float(lane_readlast(__float_as_uint(sc)));
    const bool badw = (nseg_w > 0 && !(fabsf(aw) <= 32.0f)) || !(tot <= 3.0e38f);
    if (lane == 0) {
      F.wtot[w] = tot;
      F.wflag[w] = badw ? 1u : 0u;
    }
    __syncthreads();
    float carry = 0.0f;
    bool bad = false;
    for (int i = 0; i < W; ++i) {
      if (i < w) carry += F.wtot[i];
      bad = bad || (F.wflag[i] & 1u) != 0u;
    }
    bool ex = false, fl = false;
    if (!bad && have) {
      const float incl = carry + sc;
      const float excl = carry + __uint_as_float(wave_shift_up1(__float_as_uint(sc)));
      const float lo = excl * (1.0f - DELTA), hi = incl * (1.0f + DELTA);
      const int elo = (int)(__float_as_uint(lo) >> 23) - 127;
      const int ehi = (int)(__float_as_uint(hi) >> 23) - 127;
      const bool plain = lo >= 0x1p-64f && hi <= 3.0e38f && elo == ehi;
      fl = plain && ldexpf(P.cand_theta, 23 - elo) < 2.0f;
      // EXACT: tabulate the binade the segment starts in and the next one
      int j0 = lo >= 0x1p-126f ? elo : ehi - 1;
      j0 = max(-126, min(j0, 126));
      F.sflag[seg0 + lane] = plain ? PLAIN : EXACT_PRED;
      F.sj[seg0 + lane] = (int8_t)(plain ? elo : j0);
      ex = !plain;
    }
    const uint64_t exm = __ballot(ex);
    const bool flw = __ballot(fl) != 0ull;
    __syncthreads();  // every wave has read wtot/wflag
    if (lane == 0) {
      F.wnex[w] = __popcll(exm);
      F.wflag[w] = (bad ? 1u : 0u) | (flw ? 2u : 0u);
    }
    __syncthreads();
    int before = 0;
    bool flood_any = false;
    for (int i = 0; i < W; ++i) {
      if (i < w) before += F.wnex[i];
      flood_any = flood_any || (F.wflag[i] & 2u) != 0u;
    }
    if (have) {
      const int slot = before + __popcll(exm & lt_mask);
      F.sdump[seg0 + lane] = (int8_t)(ex && slot < DCAP ? slot : -1);
    }
    if (t == 0) {
      if (bad) F.fail = 1u;
      F.flood = flood_any ? 1u : 0u;
    }
  }
  __syncthreads();
  const bool flood = F.flood != 0u;
  const float theta = flood ? kInfS : P.cand_theta;

  // ---- phase S: integer sums of PLAIN segments, four segments per step;
  // specials queued (and flushed when the queue is full)
  int qn = 0;
  // re-read the queued logits, evaluate them exactly, correct the sums
  auto flush = [&]() {
    uint32_t pos2[2];
    float v2[2], q2[2];
    bool act2[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int i = h * kWave + lane;
      act2[h] = i < qn;
      pos2[h] = act2[h] ? F.qpos[w][i] : 0u;
      q2[h] = act2[h] ? F.qq[w][i] : 0.0f;
      v2[h] = xr[pos2[h]];
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (act2[h]) {
        const int seg = (int)(pos2[h] >> 8);
        const int j = F.sj[seg];
        const GridConst gc = grid_const(j, Rw, theta);
        const uint32_t rl = __float_as_uint(fmaf(q2[h], gc.sc_lo, MAGIC)) - MAGIC_BITS;
        const float e = exact_term(v2[h], m, P.temperature, t1);
        bool tie;
        const uint32_t r = grid_round(e, j, tie);
        atomicAdd(&F.ssum[seg], r - rl);
        if (tie) F.sflag[seg] = EXACT_TIE;
        if (e >= theta) push_cand(F, Q, row, e, pos2[h]);
      }
    }
    qn = 0;
  };
  bool qovf = false;
  if (!F.fail) {
    const uint32_t flag_l = have ? (uint32_t)F.sflag[seg0 + lane] : (uint32_t)EXACT_PRED;
    const int j_l = have ? (int)F.sj[seg0 + lane] : 0;
    const GridConst gc_l = grid_const(j_l, Rw, theta);
    int seg0_s = seg0, n_s = n;
    asm volatile("" : "+s"(seg0_s), "+s"(n_s));  // recompute phase-L expressions instead of keeping them
    auto lds_q = [&](int k) {
      return *reinterpret_cast<const float4*>(&F.u.data[w][min(max(k - KV, 0), KL - 1)][lane * 4]);
    };
    for (int k0 = 0; k0 < nseg_w; k0 += 4) {
      llz_f4v qa, qb, qc, qd;  // native vectors: an array or HIP's float4 struct here ends up in scratch
      switch (k0 >> 2) {
#define LLZ_GET(i) to_v4((i) < KV ? d[(i) < KV ? (i) : 0] : lds_q(i))
#define LLZ_CASE(b)                 \
  case b:                           \
    qa = LLZ_GET(4 * (b) + 0);      \
    qb = LLZ_GET(4 * (b) + 1);      \
    qc = LLZ_GET(4 * (b) + 2);      \
    qd = LLZ_GET(4 * (b) + 3);      \
    break;
        LLZ_CASE(0) LLZ_CASE(1) LLZ_CASE(2) LLZ_CASE(3) LLZ_CASE(4) LLZ_CASE(5)
        LLZ_CASE(6) LLZ_CASE(7) LLZ_CASE(8) LLZ_CASE(9) LLZ_CASE(10) LLZ_CASE(11)
#undef LLZ_CASE
#undef LLZ_GET
        default:
          qa = to_v4(lds_q(k0 + 0));
          qb = to_v4(lds_q(k0 + 1));
          qc = to_v4(lds_q(k0 + 2));
          qd = to_v4(lds_q(k0 + 3));
      }
      uint32_t r4[4], spm = 0;
      bool pl4[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int k = k0 + s;
        const int kl = min(k, kWave - 1);
        pl4[s] = k < nseg_w && readlane_u32(flag_l, kl) == (uint32_t)PLAIN;
        const float sc_lo = readlane_f32(gc_l.sc_lo, kl);
        const float sc_hi = readlane_f32(gc_l.sc_hi, kl);
        const float tspec = readlane_f32(gc_l.tspec, kl);
        const int lim = n_s - (seg0_s + k) * SEG;  // positions lane4 + c < lim are present
        const llz_f4v qv4 = s == 0 ? qa : s == 1 ? qb : s == 2 ? qc : qd;  // s is a constant here
        const float qs[4] = {qv4.x, qv4.y, qv4.z, qv4.w};
        uint32_t acc = 0, sp = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float rlo = fmaf(qs[c], sc_lo, MAGIC);
          const float rhi = fmaf(qs[c], sc_hi, MAGIC);
          acc += __float_as_uint(rlo);
          sp |= (rlo != rhi || rhi >= tspec) ? (1u << c) : 0u;
        }
        if (lim < SEG) sp &= (1u << max(0, min(4, lim - lane4))) - 1u;  // absent positions
        if (!pl4[s]) sp = 0;
        spm |= sp << (4 * s);
        r4[s] = acc - 4u * MAGIC_BITS;
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) r4[s] = wave_sum_u32(r4[s]);
      if (lane == 0) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
          if (pl4[s]) F.ssum[seg0 + k0 + s] = r4[s];
      }
      if (__ballot(spm != 0u) != 0ull) {
        // every lane appends its own specials after those of the lanes below it
        const uint32_t my = (uint32_t)__popc(spm);
        const uint32_t incl = wave_incl_scan_op(my, 0u, [](uint32_t a, uint32_t b) { return a + b; });
        const int total = (int)lane_readlast(incl);
        if (qn + total > QCAP) flush();
        if (total > QCAP) {
          qovf = true;  // more specials in four segments than the queue holds
        } else {
          int slot = qn + (int)(incl - my);
          uint32_t rem = spm;
          while (rem != 0u) {
            const int b = __ffs(rem) - 1;
            rem &= rem - 1u;
            const int s = b >> 2, c = b & 3;
            const llz_f4v qs4 = s == 0 ? qa : s == 1 ? qb : s == 2 ? qc : qd;
            const float qv = c == 0 ? qs4.x : c == 1 ? qs4.y : c == 2 ? qs4.z : qs4.w;
            F.qpos[w][slot] = (uint32_t)((seg0 + k0 + s) * SEG + lane4 + c);
            F.qq[w][slot] = qv;
            ++slot;
          }
          qn += total;
        }
      }
    }
    if (qovf && lane == 0) atomicOr(&F.fail, 1u);
  }

  // ---- phase F+X: the remaining specials and the first EXACT slots in one
  // round trip (the slots overlay the LDS-resident segments: every wave is
  // past phase S)
  __syncthreads();
  if (!F.fail) {
    uint32_t pos2[2];
    float v2[2], q2[2];
    bool act2[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int i = h * kWave + lane;
      act2[h] = i < qn;
      pos2[h] = act2[h] ? F.qpos[w][i] : 0u;
      q2[h] = act2[h] ? F.qq[w][i] : 0.0f;
      v2[h] = xr[pos2[h]];
    }
    const uint64_t emask = exact_mask(F, seg0, nseg_w, 0);
    exact_loads<FASTLD>(F, xr, seg0, emask, n);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (act2[h]) {
        const int seg = (int)(pos2[h] >> 8);
        const int j = F.sj[seg];
        const GridConst gc = grid_const(j, Rw, theta);
        const uint32_t rl = __float_as_uint(fmaf(q2[h], gc.sc_lo, MAGIC)) - MAGIC_BITS;
        const float e = exact_term(v2[h], m, P.temperature, t1);
        bool tie;
        const uint32_t r = grid_round(e, j, tie);
        atomicAdd(&F.ssum[seg], r - rl);
        if (tie) F.sflag[seg] = EXACT_TIE;
        if (e >= theta) push_cand(F, Q, row, e, pos2[h]);
      }
    }
    exact_segments(F, Q, P, row, seg0, emask, n, m, theta, t1);
  }
  __syncthreads();

  // ---- phase C: the walk in index order; later EXACT segments in rounds
  for (int round = 0; !F.fail; ++round) {
    const int g_from = F.next_g;
    if (round > 0) {
      if (w == 0) {  // slots for the EXACT segments from g_from on, in order
        int cnt = 0;
        for (int b = g_from; b < G; b += kWave) {
          const int g = b + lane;
          const bool ex = g < G && F.sflag[g] != PLAIN;
          const uint64_t mk = __ballot(ex);
          const int slot = cnt + __popcll(mk & lt_mask);
          if (ex) {
            F.sdump[g] = (int8_t)(slot < DCAP ? slot : -1);
          }
          cnt += __popcll(mk);
        }
      }
      __syncthreads();
      const uint64_t emask = exact_mask(F, seg0, nseg_w, g_from);
      exact_loads<FASTLD>(F, xr, seg0, emask, n);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      exact_segments(F, Q, P, row, seg0, emask, n, m, theta, t1);
      __syncthreads();
    }
    if (w == 0) {
      float s = F.s_run;
      int g = g_from;
      bool fail = false, more = false;
      while (g < G) {
        const Grid gr = grid_of(s);
        const int gg = g + lane;
        bool okp = false;
        uint32_t sm = 0;
        if (gg < G) {
          okp = F.sflag[gg] == PLAIN && (int)F.sj[gg] == gr.j;
          sm = F.ssum[gg];
        }
        const uint64_t bad = __ballot(!okp);
        const int fb = bad ? __ffsll((long long)bad) - 1 : kWave;
        const uint32_t incl = wave_incl_scan_sat(lane < fb ? sm : 0u, kSat);
        if (__ballot(lane < fb && gr.N + incl >= kGridTop) != 0ull) {
          fail = true;  // a crossing the prediction did not see
          break;
        }
        if (fb > 0) {
          s = grid_value(gr.N + readlane_u32(incl, fb - 1), gr.j);
          g += fb;
        }
        if (fb < kWave && g < G) {
          if (F.sflag[g] == PLAIN) {
            fail = true;  // the running sum is not in the predicted binade
            break;
          }
          const int slot = F.sdump[g];
          if (slot < 0 || g < g_from) {
            more = true;
            break;
          }
          s = resolve_exact(s, slot, F.sj[g], F);
          ++g;
        }
      }
      if (lane == 0) {
        F.s_run = s;
        F.next_g = g;
        if (fail) F.fail = 1u;
        F.done = (!fail && !more) ? 1 : 0;
      }
    }
    __syncthreads();
    if (F.done) break;
  }

  if (t == 0) {
    if (!F.fail) {
      rs_out[0] = m;
      rs_out[1] = F.s_run;
      rs_out[2] = __uint_as_float(flood ? (uint32_t)kCandCap + 1u : F.ncand);
      rs_out[3] = 0.0f;
    } else {
      // not certified: k_select runs the streaming normaliser on this row
      rs_out[0] = m;
      rs_out[1] = 0.0f;
      rs_out[2] = __uint_as_float(0u);
      rs_out[3] = 1.0f;
    }
  }
}

}  // namespace

hipError_t launch_stats(const RowParams& P, const RowPtrs& Q, hipStream_t st) {
  if ((P.flags & kFlagVecSrc) != 0 && (P.n % 4) == 0)
    hipLaunchKernelGGL(k_stats<true>, dim3(P.rows), dim3(NT), 0, st, P, Q);
  else
    hipLaunchKernelGGL(k_stats<false>, dim3(P.rows), dim3(NT), 0, st, P, Q);
  return hipGetLastError();
}

}  // namespace llz
