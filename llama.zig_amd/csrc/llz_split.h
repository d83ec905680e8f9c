// llz_split.h -- token-only rows of small batches read by several workgroups.
//
// One workgroup per row (k_stats) leaves most CUs idle when a call holds few
// rows, and a single CU reads a 128K-logit row at a fraction of the chip's
// bandwidth.  Here row r's logits are cut into S chunks of 2048 nv
// consecutive positions, one workgroup each (grid rows x S).  Each chunk
// workgroup computes
//   m_c  its maximum (NaNs skipped, as sampler.zig:80-81 skips them),
//   c_c  = RN(m_c l2e_t), and s_c = sum of exp2(fma(v, l2e_t, -c_c)), the
//        estimates of phase L of k_stats taken against the chunk's maximum,
//   its list: at most kSplitK elements that may be candidates, as (logit,
//        position), and vt, the largest logit of those it left out.
// The elements that may be candidates are those with d2 = (m_c - v) l2e_t
// below B = log2(1 / theta) + 2^-8 (theta = tok_theta): with m >= m_c the
// row's maximum, an element outside has a term exp((v - m) / T) below theta
// 2^-(2^-8) (1 + 2^-19) < theta, whatever m.  When more than kSplitK lie
// below B, a 256-bin histogram of d2 over [0, B) picks the longest prefix
// of bins holding at most kSplitK of them.
//
// The workgroup that publishes the row's last chunk merges: every chunk
// workgroup publishes its list and summary, then its tag (the call's epoch),
// then reads the others' tags; one that sees all S takes the row with a
// compare-and-swap.  The records travel between workgroups on different
// XCDs, whose L2 caches are not coherent with each other: every access to
// them is a relaxed agent-scope atomic, which the hardware performs at the
// device's point of coherence (no stale copy in a CU's or an XCD's cache),
// and the order is kept by waiting for the stores' completion (vmcnt 0)
// before the next step's stores or loads are issued:
//   list and summary stores, complete -> tag store, complete -> tag loads;
//   tag loads returned -> (elected) the merge's loads.
// The last workgroup to complete its tag store sees every tag: any other's
// tag store completed before that workgroup's tag loads were issued, or
// after it, and then that other workgroup's own loads see this tag.  (A
// release fence at agent scope would write back the whole L2 of each
// workgroup's XCD, microseconds per workgroup.)
//
//   m = max m_c; the normaliser's estimate sum_c s_c exp2(fma(m, -l2e_t,
//   c_c)) (the chunk sums scaled to the row's maximum, as phase M scales
//   the waves' sums); the list: the chunks' entries whose exact term
//   (sampler.zig:85) reaches theta.  The list is complete when every chunk's
//   vt has a term below theta (1 - 2^-21): exp_f32 is within an ulp of exp,
//   so no logit below vt has a term above that of vt by more than 2^-22.
// token_select then makes the chain's decisions exactly as for a row of
// k_stats's token path.  A row that any check fails (a NaN, an infinite
// maximum, an incomplete or overlong list, an undecided decision) is
// finished by the merging workgroup with k_stats's full single-row path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "llz_fast.h"
#include "llz_internal.h"
#include "llz_norm.h"
#include "llz_select.h"
#include "llz_token.h"
#include "llz_wg.h"
#include "llz_xform.h"

namespace llz {

constexpr int kSplitNT = fastp::NT;  // threads of a chunk workgroup (k_stats's, whose single-row path it may run)
constexpr int kSplitW = kSplitNT / kWave;
constexpr int kSplitSeg = kSplitNT * 4;  // logits per float4 step of a chunk workgroup
constexpr int kSplitBins = 256;
constexpr int kSplitStampRow = 2048;  // measurement builds: chunk workgroup b stamps row kSplitStampRow + b

struct SplitShared {
  uint32_t hist[kSplitBins];
  float wm[kSplitW];
  uint32_t wnan[kSplitW];
  float ws[kSplitW];
  float wws[kSplitW];  // per wave: its estimates times n - their position
  float wvt[kSplitW];
  uint32_t win[kSplitW];    // elements below B per wave
  unsigned long long lst[kSplitK];  // the chunk's list, staged for wave 0's stores
  uint32_t pen[kPenMax];  // the penalised positions in this chunk (fused penalty)
  uint32_t npen;
  uint32_t ncoll;     // entries written to the chunk's list
  uint32_t nb;        // bins collected
  uint32_t elected;   // this workgroup saw every chunk published (then: took the row's full path)
  // the merge
  uint64_t tl[2 * kTokCap];  // collected, then sorted
  uint8_t part[kSplitW * kTokCap];
  uint32_t ncv[kSplitMax];   // per chunk: its list entries that may pass (0: none)
  uint32_t tcand, tfail, bad;
  float m, s_est, w_est;
};

// Device-coherent accesses to the split records, and the wait for this
// wave's stores to complete.
__device__ __forceinline__ void dev_st(unsigned long long* p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long dev_ld(unsigned long long* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stores_done() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ unsigned long long pack2(float lo, float hi) {
  return (unsigned long long)__float_as_uint(lo) | ((unsigned long long)__float_as_uint(hi) << 32);
}
__device__ __forceinline__ float lo_f(unsigned long long w) { return __uint_as_float((uint32_t)w); }
__device__ __forceinline__ float hi_f(unsigned long long w) { return __uint_as_float((uint32_t)(w >> 32)); }

__device__ __forceinline__ float4 split_ld4(const float* xr, int pos, int n) {
  const bool in = pos < n;
  const float4 v = ld_nt4(xr + (in ? pos : 0));
  const float ni = -__builtin_inff();
  return in ? v : make_float4(ni, ni, ni, ni);
}

// Chunk c of row `row` (every thread of the workgroup), NV = split_nv float4
// per thread (a template parameter: the loads, all issued at once, need no
// branch between them).  XF: the row is read through the caller's
// post-processing and the fused repetition penalty (P.xf_src), applied
// exactly to every logit of the chunk as it lands (a few per thread).
// Returns true in every thread of a workgroup that saw every chunk of the
// row published and goes on to merge it.
template <int NV, bool XF>
__device__ __forceinline__ bool split_chunk(const KArgs& A, int row, int c, SplitShared& S) {
  const RowParams& P = A.P;
  const RowPtrs& Q = A.Q;
  const int t = (int)threadIdx.x, lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(wave_id());
  const int n = P.n;
  const int base = c * (kSplitSeg * NV);
  const float* xr = Q.src + (int64_t)row * P.src_stride;
  SplitRow& R = Q.split[row];
  const int sr = kSplitStampRow + (int)blockIdx.x;  // measurement builds: this workgroup's stamp row
  (void)sr;
  LLZ_STAMP(sr, 0);
  // every load in flight at once (step j: the workgroup's 2048 logits from
  // base + 2048 j, one float4 per thread)
  float4 v[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) v[j] = split_ld4(xr, base + (j * kSplitNT + t) * 4, n);  // absent: -inf
  if constexpr (XF) {
    const uint32_t xf = P.xf_src;
    // main.zig:653-666 on each logit of the row (positions past it stay -inf)
    if (xf & (kXfCap | kXfScale)) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int pos = base + (j * kSplitNT + t) * 4;
        v[j].x = pos + 0 < n ? logit_post(v[j].x, xf, P.cap, P.inv_scale) : v[j].x;
        v[j].y = pos + 1 < n ? logit_post(v[j].y, xf, P.cap, P.inv_scale) : v[j].y;
        v[j].z = pos + 2 < n ? logit_post(v[j].z, xf, P.cap, P.inv_scale) : v[j].z;
        v[j].w = pos + 3 < n ? logit_post(v[j].w, xf, P.cap, P.inv_scale) : v[j].w;
      }
    }
    // sampler.zig:54-75: each distinct id < n of the window (lane j of wave
    // 0 holds id j) that lies in this chunk, penalised by the thread that
    // holds it
    if (xf & kXfPen) {
      if (w == 0) {
        const uint32_t id = pen_window_id(P, Q, row);
        bool first = id < (uint32_t)n;
        for (int j = 0; j < P.pen_w; ++j) {
          const uint32_t o = readlane_u32(id, j);
          first = first && !(j < lane && o == id);
        }
        const bool mine = first && id >= (uint32_t)base && id - (uint32_t)base < (uint32_t)(kSplitSeg * NV);
        const uint64_t bm = bal64(mine);
        const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
        if (mine) S.pen[__popcll(bm & lt)] = id;
        if (lane == 0) S.npen = (uint32_t)__popcll(bm);
      }
      lds_barrier();
      const int np = (int)S.npen;
      for (int i = 0; i < np; ++i) {
        const uint32_t rel = S.pen[i] - (uint32_t)base;
        const int jj = (int)(rel / kSplitSeg), q = (int)(rel % kSplitSeg);
        if ((q >> 2) == t) {
          const int k = q & 3;
#pragma unroll
          for (int j = 0; j < NV; ++j) {
            v[j].x = j == jj && k == 0 ? penalise(v[j].x, P.rpen) : v[j].x;
            v[j].y = j == jj && k == 1 ? penalise(v[j].y, P.rpen) : v[j].y;
            v[j].z = j == jj && k == 2 ? penalise(v[j].z, P.rpen) : v[j].z;
            v[j].w = j == jj && k == 3 ? penalise(v[j].w, P.rpen) : v[j].w;
          }
        }
      }
    }
  }
  if (t < kSplitBins) S.hist[t] = 0u;
  if (t == 0) S.ncoll = 0u;
  float mx = -__builtin_inff();
  uint32_t nanf = 0u;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    mx = fmaxf(fmaxf(mx, fmaxf(v[j].x, v[j].y)), fmaxf(v[j].z, v[j].w));  // fmaxf skips NaN
    nanf |= (uint32_t)((v[j].x != v[j].x) | (v[j].y != v[j].y) | (v[j].z != v[j].z) | (v[j].w != v[j].w));
  }
  mx = wave_max_f32(mx);
  const bool wn = bal64(nanf != 0u) != 0ull;
  if (lane == 0) {
    S.wm[w] = mx;
    S.wnan[w] = wn ? 1u : 0u;
  }
  lds_barrier();
  LLZ_STAMP(sr, 1);
  float mc = -__builtin_inff();
  bool nan = false;
#pragma unroll
  for (int i = 0; i < kSplitW; ++i) {
    mc = fmaxf(mc, S.wm[i]);
    nan = nan || S.wnan[i] != 0u;
  }
  const bool special = nan || mc > 3.0e38f;
  const float l2e = P.l2e_t;
  const float cc = fabsf(mc) <= 3.0e38f ? mc * l2e : 0.0f;
  const float B = P.split_b, bs = P.split_bs;
  // the estimates' sum, and the elements below B: counted, then (when more
  // than kSplitK) binned
  float s = 0.0f, sw = 0.0f;
  uint32_t cin = 0u;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const float4 x = v[j];
    const float q0 = __builtin_amdgcn_exp2f(fmaf(x.x, l2e, -cc));
    const float q1 = __builtin_amdgcn_exp2f(fmaf(x.y, l2e, -cc));
    const float q2 = __builtin_amdgcn_exp2f(fmaf(x.z, l2e, -cc));
    const float q3 = __builtin_amdgcn_exp2f(fmaf(x.w, l2e, -cc));
    s += (q0 + q1) + (q2 + q3);
    // weighted by n - pos (the interval of S, llz_token.h): absent
    // positions have q = 0
    const float rem = (float)(n - (base + (j * kSplitNT + t) * 4));
    sw += (q0 * rem + q1 * (rem - 1.0f)) + (q2 * (rem - 2.0f) + q3 * (rem - 3.0f));
    cin += (uint32_t)(((mc - x.x) * l2e < B) + ((mc - x.y) * l2e < B) + ((mc - x.z) * l2e < B) +
                      ((mc - x.w) * l2e < B));
  }
  const uint32_t win = wave_sum_u32(cin);
  if (lane == 0) S.win[w] = win;
  lds_barrier();
  LLZ_STAMP(sr, 2);
  uint32_t tin = 0u;
#pragma unroll
  for (int i = 0; i < kSplitW; ++i) tin += S.win[i];
  auto bin_of = [&](float d2) { return min(kSplitBins - 1, (int)(d2 * bs)); };
  uint32_t nb = kSplitBins;
  if (tin > (uint32_t)kSplitK) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const float xs[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float d2 = (mc - xs[k]) * l2e;
        if (d2 < B) atomicAdd(&S.hist[bin_of(d2)], 1u);
      }
    }
    lds_barrier();
    if (w == 0) {
      // bins 4 lane .. 4 lane + 3; nb = the bins whose inclusive count is at
      // most kSplitK (a prefix: the counts do not decrease)
      uint32_t h[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) h[k] = S.hist[4 * lane + k];
      const uint32_t loc = (h[0] + h[1]) + (h[2] + h[3]);
      uint32_t run = wave_incl_scan_op(loc, 0u, [](uint32_t a, uint32_t b) { return a + b; }) - loc;
      uint32_t cnt = 0u;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        run += h[k];
        cnt += run <= (uint32_t)kSplitK ? 1u : 0u;
      }
      const uint32_t tot = wave_sum_u32(cnt);
      if (lane == 0) S.nb = tot;
    }
    lds_barrier();
    nb = S.nb;
    LLZ_STAMP(sr, 3);
  }
  // the list: elements of bins below nb; vt: the largest other element below B
  auto taken = [&](float d2) { return d2 < B && (nb == (uint32_t)kSplitBins || bin_of(d2) < (int)nb); };
  float vt = -__builtin_inff();
  uint32_t pc = 0u;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const float xs[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float d2 = (mc - xs[k]) * l2e;
      const bool take = taken(d2);
      pc += take ? 1u : 0u;
      vt = d2 < B && !take ? fmaxf(vt, xs[k]) : vt;
    }
  }
  const uint32_t pin = wave_incl_scan_op(pc, 0u, [](uint32_t a, uint32_t b) { return a + b; });
  const uint32_t wtot = readlane_u32(pin, kWave - 1);
  uint32_t wbase = 0u;
  if (lane == 0 && wtot != 0u) wbase = atomicAdd(&S.ncoll, wtot);
  uint32_t slot = readlane_u32(wbase, 0) + pin - pc;
  if (pc != 0u) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const float xs[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const bool take = taken((mc - xs[k]) * l2e);
        if (take && slot < (uint32_t)kSplitK)
          S.lst[slot] = (unsigned long long)__float_as_uint(xs[k]) |
                        ((unsigned long long)(base + (j * kSplitNT + t) * 4 + k) << 32);
        slot += take ? 1u : 0u;
      }
    }
  }
  const float ws = wave_sum_f32(s);
  const float wws = wave_sum_f32(sw);
  vt = wave_max_f32(vt);
  if (lane == 0) {
    S.ws[w] = ws;
    S.wws[w] = wws;
    S.wvt[w] = vt;
  }
  lds_barrier();
  LLZ_STAMP(sr, 4);
  // wave 0 publishes: the list (one store per lane) and the summary, then,
  // once they are complete, the tag
  if (w == 0) {
    const uint32_t ncoll = S.ncoll;
    if ((uint32_t)lane < ncoll) dev_st(&R.cand[c * kSplitK + lane], S.lst[lane]);
    if (lane == 0) {
      SplitRec& rc = R.rec[c];
      const float sum = ((S.ws[0] + S.ws[1]) + (S.ws[2] + S.ws[3])) + ((S.ws[4] + S.ws[5]) + (S.ws[6] + S.ws[7]));
      const float wsum =
          ((S.wws[0] + S.wws[1]) + (S.wws[2] + S.wws[3])) + ((S.wws[4] + S.wws[5]) + (S.wws[6] + S.wws[7]));
      float vm = S.wvt[0];
#pragma unroll
      for (int i = 1; i < kSplitW; ++i) vm = fmaxf(vm, S.wvt[i]);
      dev_st(&rc.mc, pack2(mc, cc));
      dev_st(&rc.sv, pack2(sum, vm));
      dev_st(&rc.nf, (unsigned long long)(ncoll | (special ? 0x10000u : 0u)) |
                         ((unsigned long long)__float_as_uint(wsum) << 32));
    }
    stores_done();  // the list and the summary complete
    if (lane == 0) {
      dev_st(&R.rec[c].tag, (unsigned long long)P.epoch);
      stores_done();  // the tag before the reads of the others'
      LLZ_STAMP(sr, 5);
    }
    const int ns = P.split_s;
    const unsigned long long tg = lane < ns ? dev_ld(&R.rec[lane].tag) : P.epoch;
    const bool all = bal64(tg != P.epoch) == 0ull;
    if (lane == 0) S.elected = all ? 1u : 0u;
  }
  __syncthreads();
  LLZ_STAMP(sr, 6);
  return S.elected != 0u;
}

// One workgroup of those that saw row `row`'s chunks published takes the
// row (compare-and-swap of the row's word to the call's epoch); true in
// every thread of that one.
__device__ __forceinline__ bool split_take(const KArgs& A, int row, SplitShared& S) {
  SplitRow& R = A.Q.split[row];
  if (threadIdx.x == 0) {
    uint32_t el = 0u;
    unsigned long long cur = dev_ld(&R.elect);
    if (cur != A.P.epoch)
      el = __hip_atomic_compare_exchange_strong(&R.elect, &cur, (unsigned long long)A.P.epoch, __ATOMIC_RELAXED,
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
               ? 1u
               : 0u;
    S.elected = el;
  }
  __syncthreads();
  return S.elected != 0u;
}

// The merge (every thread of a workgroup that saw the row's chunks
// published).  Returns true when it finished the row (outputs written),
// false when the row is not certified.  Two workgroups may both merge a row
// (k_split merges before taking the row, to save a round trip): they read
// the same final records and write the same outputs.
__device__ __forceinline__ bool split_merge(const KArgs& A, int row, SplitShared& S) {
  const RowParams& P = A.P;
  const RowPtrs& Q = A.Q;
  const int t = (int)threadIdx.x, lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(wave_id());
  SplitRow& R = Q.split[row];
  const float T = P.temperature, theta = P.tok_theta, l2e = P.l2e_t;
  const bool t1 = (P.flags & kFlagTIsOne) != 0u;
  const float u_row = Q.uniforms[row];
  const float ninf = -__builtin_inff();
  const int ns = P.split_s;
  const int sr = kSplitStampRow + (int)blockIdx.x;
  (void)sr;
  LLZ_STAMP(sr, 7);
  // every thread: its share of the chunks' list slots, loaded with the
  // summaries in one round trip (slots past a chunk's count hold words of
  // other calls: dropped below)
  constexpr int kPer = kSplitMax * kSplitK / kSplitNT;
  const int nslots = ns * kSplitK;
  unsigned long long en[kPer];
#pragma unroll
  for (int h = 0; h < kPer; ++h) {
    const int i = h * kSplitNT + t;
    en[h] = dev_ld(&R.cand[i < nslots ? i : 0]);
  }
  if (w == 0) {
    const bool on = lane < ns;
    float mc = ninf, cc = 0.0f, sc = 0.0f, vt = ninf, wc = 0.0f;
    uint32_t nc = 0u, fl = 0u;
    if (on) {
      SplitRec& rc = R.rec[lane];
      const unsigned long long a = dev_ld(&rc.mc), b = dev_ld(&rc.sv), d = dev_ld(&rc.nf);
      mc = lo_f(a);
      cc = hi_f(a);
      sc = lo_f(b);
      vt = hi_f(b);
      nc = (uint32_t)d & 0xffffu;
      fl = ((uint32_t)d >> 16) & 1u;
      wc = hi_f(d);
    }
    const float m = wave_max_f32(mc);
    bool bad = fl != 0u || !(fabsf(m) <= 3.0e38f) || nc > (uint32_t)kSplitK;
    // the chunk sums scaled to the row's maximum (aw <= 0 up to roundings;
    // a chunk far below the maximum adds less than 2^-64 of its sum, whose
    // loss is far inside the normaliser's interval)
    const bool live = on && mc > ninf;
    const float aw = fmaf(m, -l2e, cc);
    bad = bad || (live && !(aw <= 1.0f));
    const float rc = __builtin_amdgcn_exp2f(aw);
    const float s_est = wave_sum_f32(live ? sc * rc : 0.0f);
    const float w_est = wave_sum_f32(live ? wc * rc : 0.0f);
    bool inc = false;
    if (live && !bad) {
      // completeness: the chunk's left-out elements stay below theta
      if (vt > ninf && !(exact_term(vt, m, T, t1) * (1.0f + 0x1p-21f) < theta)) bad = true;
      // a chunk whose maximum's term is below theta holds no candidate
      inc = nc > 0u && !(exact_term(mc, m, T, t1) * (1.0f + 0x1p-21f) < theta);
    }
    S.ncv[lane] = inc ? nc : 0u;
    const bool any_bad = bal64(bad) != 0ull;
    if (lane == 0) {
      S.bad = any_bad ? 1u : 0u;
      S.m = m;
      S.s_est = s_est;
      S.w_est = w_est;
      S.tcand = 0u;
      S.tfail = 0u;
    }
  }
  lds_barrier();
  LLZ_STAMP(sr, 8);
  bool ok = S.bad == 0u;
  if (ok) {
    const float m = S.m;
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
#pragma unroll
    for (int h = 0; h < kPer; ++h) {
      const int i = h * kSplitNT + t;
      const bool live = i < nslots && (uint32_t)(i % kSplitK) < S.ncv[i / kSplitK];
      if (bal64(live) == 0ull) continue;  // most slots belong to chunks that hold no candidate
      const float e = live ? exact_term(lo_f(en[h]), m, T, t1) : 0.0f;  // sampler.zig:85
      const bool cand = live && e >= theta;
      const uint64_t cb = bal64(cand);
      if (cb != 0ull) {
        uint32_t b0 = 0u;
        if (lane == 0) b0 = atomicAdd(&S.tcand, (uint32_t)__popcll(cb));
        const uint32_t sl = readlane_u32(b0, 0) + (uint32_t)__popcll(cb & lt);
        if (cand && sl < (uint32_t)kTokCap) S.tl[sl] = ((uint64_t)(~__float_as_uint(e)) << 32) | (uint32_t)(en[h] >> 32);
      }
    }
    lds_barrier();
    LLZ_STAMP(sr, 9);
    const int tc = (int)S.tcand;
    ok = tc <= kTokCap;
    if (ok) {
      token_sort(S.tl, S.tl + kTokCap, S.part, tc);
      if (w == 0) token_select<false>(kernel_args_ptr(), row, S.tl + kTokCap, tc, S.s_est, S.w_est, 0.0, -1.0, u_row, theta, &S.tfail);
      lds_barrier();
      LLZ_STAMP(sr, 10);
      ok = S.tfail == 0u;
    }
  }
  if (ok && t == 0 && Q.status) Q.status[row] = kPathTokenOnly | kPathSplit;  // after token_select's store (same thread)
  return ok;
}

}  // namespace llz
