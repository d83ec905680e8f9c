// llz_bucket.h -- top-k / top-p / min-p, the total and the draw
// (sampler.zig:106-126, 156-168) for a row whose kept prefix is longer than
// the candidate list, without sorting the row.
//
// The chain reads the row in the order (p desc, id asc).  Top-k, top-p and
// min-p keep a prefix of that order; the total is the sequential f32 sum of
// the prefix; the draw subtracts the prefix's terms from u * total until the
// value reaches 0.  Keys k = ~bits(p) ascend in that order, so the order is
// (k asc, id asc), and buckets of consecutive key ranges hold consecutive
// runs of it.
//
// While a sequential f32 sum stays in one binade [2^j, 2^(j+1)) its grid is
// u = 2^(j-23) and every term adds RN(p / u) units, whatever the order of the
// terms (llz_exact.h), unless a term is a tie.  The same holds for the
// draw's subtractions while the value stays above 2^j.  So a bucket whose
// running value is predicted to stay inside one binade (PLAIN) contributes
// one integer sum, accumulated in any order; only the buckets where the
// value may cross a binade boundary, where the top-p cut or the kept prefix's
// end may fall, where the draw may stop, or that hold a tie (EXACT) need
// their elements in order: they are gathered, sorted in LDS, and taken term
// by term.  The walks check every prediction (the value must leave a PLAIN
// bucket on its grid); a row whose check fails, or whose EXACT buckets hold
// too many elements, returns false and takes the sorting path.
//
// Passes over the row (one workgroup):
//   A  the exact p of every element (the reference's operations), its key
//      written to the fallback buffer; a coarse histogram of the keys
//      (count and mass) locates the region the chain can reach;
//   A' a fine histogram of that region from the stored keys;
//   B  (per walk) the PLAIN buckets' integer sums on their grids and the
//      EXACT buckets' elements; B2 gathers buckets a tie made EXACT.
#pragma once

#include "llz_accum.h"
#include "llz_rowops.h"

namespace llz {

constexpr int kNB = 4096;          // fine buckets
constexpr int kBList = 4096;       // gathered (EXACT) elements per walk at most
constexpr int kCoarseShift = 17;   // coarse histogram: 2^17 keys per bucket
constexpr int kBucketMinN = 8192;  // shorter rows keep the sorting path
// Relative margin of the predictions: the exact running value differs from
// the histogram's real-valued prefix by the sequential rounding (about
// sqrt(count / 12) units of the running value's grid on random data: 9e-6
// relative after configuration 4's 217k terms, so 2^-16 declined 3% of its
// rows), the truncation of lower-binade terms in the bucket masses and their
// f32 rounding (each about 2^-24).
constexpr double kBucketDelta = 0x1p-13;
constexpr int kCountShift = 44;  // histogram word: count << 44 | sum of scaled significands
// Bucket arrays are padded by one entry per 64 buckets: wave 0's scans give
// each lane 64 consecutive buckets, which unpadded would sit in one LDS bank.
constexpr int kNBP = kNB + kNB / 64;
__device__ __forceinline__ int bix(int b) { return b + (b >> 6); }

enum : uint8_t { kBNone = 0, kBEmpty = 1, kBPlain = 2, kBExact = 3, kBExactTie = 4 };

struct BucketShared {  // arrays indexed through bix()
  uint32_t cnt[kNBP];   // elements per bucket
  float mass[kNBP];     // their p summed (predictions only)
  union {
    struct {
      uint32_t sum[kNBP];  // PLAIN: integer sum of RN(p / u) on grid jg
      uint32_t off[kNBP];  // EXACT: first position in the sorted list
    };
    uint64_t hist[kNBP];   // histogram passes: count << 44 | the significands of p scaled to the bucket's top binade
  };
  int8_t jg[kNBP];      // PLAIN: the binade of the running value
  uint8_t cls[kNBP];
  uint8_t tie[kNBP];    // PLAIN: bit 0 a term is a tie on grid jg, bit 1 the sum reached kSat
  uint64_t list[kBList];  // EXACT buckets' elements, (key << 32 | id), sorted
  uint32_t nlist;
  uint32_t ctl[8];
};

struct BucketResult {
  uint32_t K;       // kept prefix length
  float total;      // sampler.zig:156-159
  uint32_t token;
  uint32_t consumed;
  uint32_t why;     // the bucket path declined: 1 + step (diagnostic, status bits 8-15)
};

// Eight stored keys from pos (absent positions: 0xffffffff, which no bucket
// range holds).
__device__ __forceinline__ void bucket_keys8(const uint32_t* Kp, int pos, int n, uint32_t (&k)[8]) {
  if (pos + 8 <= n && (reinterpret_cast<uintptr_t>(Kp + pos) & 15u) == 0u) {
    const uint4 a = *reinterpret_cast<const uint4*>(Kp + pos);
    const uint4 b = *reinterpret_cast<const uint4*>(Kp + pos + 4);
    k[0] = a.x; k[1] = a.y; k[2] = a.z; k[3] = a.w;
    k[4] = b.x; k[5] = b.y; k[6] = b.z; k[7] = b.w;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) k[i] = pos + i < n ? Kp[pos + i] : 0xffffffffu;
  }
}

__device__ __forceinline__ float key_p(uint32_t key) { return __uint_as_float(~key); }

// Biased exponent of p = key_p(key) (1 for subnormals) and its 24-bit
// significand: p = sig * 2^(E - 150).
__device__ __forceinline__ uint32_t key_E(uint32_t key) {
  const uint32_t e = (~key >> 23) & 0xffu;
  return e == 0u ? 1u : e;
}
__device__ __forceinline__ uint32_t key_sig(uint32_t key) {
  const uint32_t b = ~key;
  return (b & 0x7fffffu) | (((b >> 23) & 0xffu) != 0u ? 0x800000u : 0u);
}

// One element's histogram word for a bucket whose largest p has biased
// exponent Etop: its count and its significand scaled to 2^(Etop - 150)
// (terms of lower binades lose their low bits: relative error < 2^-23 each).
__device__ __forceinline__ uint64_t hist_word(uint32_t key, uint32_t Etop) {
  const uint32_t d = Etop - key_E(key);  // >= 0: p <= the bucket's largest
  const uint64_t v = d < 24u ? (uint64_t)(key_sig(key) >> d) : 0ull;
  return (1ull << kCountShift) | v;
}

// Count and mass of a bucket from its histogram word (Etop as above).
__device__ __forceinline__ void hist_unpack(uint64_t h, uint32_t Etop, uint32_t& cnt, float& mass) {
  cnt = (uint32_t)(h >> kCountShift);
  const double sig = (double)(h & ((1ull << kCountShift) - 1ull));
  mass = (float)(sig * exp2((double)((int)Etop - 150)));
}

// Binade of a positive double (its unbiased exponent; -1023 for 0).
__device__ __forceinline__ int dbl_binade(double x) {
  return (int)((uint64_t)__double_as_longlong(x) >> 52 & 0x7ffu) - 1023;
}

// A wave's sequential chain over len terms (sampler.zig:112-117 / :162-166):
// ADD stops at the first value > thr (thr >= 0), SUB at the first value <= 0.
// Returns the value after the stopping term (or after the last), with
// `before` the value before the stopping term.
template <bool SUB, typename TermFn>
__device__ float wave_seq_stop(float s, int len, float thr, int& stop, float& before, TermFn term) {
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
      before = L > 0 ? readlane_f32(acc, L - 1) : s;
      return readlane_f32(acc, L);
    }
    s = readlane_f32(acc, cnt - 1);
  }
  before = s;
  return s;
}

// Wave 0: exclusive prefixes of the buckets' counts and masses, 64 buckets a
// lane; calls cls_of(b, excl_count, excl_mass) for every bucket in order
// within the lane.
template <typename ClsFn>
__device__ __forceinline__ void bucket_scan(BucketShared& bs, ClsFn cls_of) {
  constexpr int PL = kNB / kWave;
  const int lane = lane_id();
  uint32_t c = 0;
  double ms = 0.0;
  for (int i = 0; i < PL; ++i) {
    c += bs.cnt[bix(lane * PL + i)];
    ms += (double)bs.mass[bix(lane * PL + i)];
  }
  uint32_t ci = c;
  double mi = ms;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t oc = __shfl_up(ci, d, kWave);
    const double om = __shfl_up(mi, d, kWave);
    if (lane >= d) {
      ci += oc;
      mi += om;
    }
  }
  uint32_t ec = ci - c;
  double em = mi - ms;
  for (int i = 0; i < PL; ++i) {
    const int b = lane * PL + i;
    cls_of(b, ec, em);
    ec += bs.cnt[bix(b)];
    em += (double)bs.mass[bix(b)];
  }
}

// Bucket of a key in the fine range [kmin, kcut): (key - kmin) >> shift.
struct BucketRange {
  uint32_t kmin, kcut;
  int shift;
  __device__ __forceinline__ bool in(uint32_t key) const { return key >= kmin && key < kcut; }
  __device__ __forceinline__ int of(uint32_t key) const { return (int)min((key - kmin) >> shift, (uint32_t)kNB - 1u); }
};

// Pass B: the PLAIN buckets' integer sums of RN(p / u) on their grids, with
// tie and saturation flags; then a bucket holding a tie becomes EXACT and one
// whose sum saturated (a wrong prediction) NONE, where a walk stops.
template <int NT>
__device__ void bucket_sums(const uint32_t* Kp, int n, const BucketRange& br, BucketShared& bs) {
  const int t = (int)threadIdx.x;
  for (int b = t; b < kNB; b += NT) {
    bs.sum[bix(b)] = 0u;
    bs.tie[bix(b)] = 0u;
  }
  __syncthreads();
  for (int base = 0; base < n; base += NT * 8) {
    const int pos = base + t * 8;
    uint32_t k[8];
    bucket_keys8(Kp, pos, n, k);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (!br.in(k[i])) continue;
      const int b = br.of(k[i]);
      if (bs.cls[bix(b)] == kBPlain) {
        bool tie;
        const uint32_t r = grid_round(key_p(k[i]), bs.jg[bix(b)], tie);  // <= kSat
        // terms <= kSat and a flag once the sum reaches kSat: no wrap goes unseen
        const uint32_t old = atomicAdd(&bs.sum[bix(b)], r);
        if (tie) bs.tie[bix(b)] |= 1u;
        if (old >= kSat) bs.tie[bix(b)] |= 2u;
      }
    }
  }
  __syncthreads();
  for (int b = t; b < kNB; b += NT) {
    if (bs.cls[bix(b)] == kBPlain && (bs.tie[bix(b)] & 2u))
      bs.cls[bix(b)] = kBNone;
    else if (bs.cls[bix(b)] == kBPlain && bs.tie[bix(b)])
      bs.cls[bix(b)] = kBExact;
  }
  __syncthreads();
}

// The EXACT buckets from `blo` on whose elements fit the list together:
// gathered, sorted, and each bucket's place in the list.  Returns the end of
// that bucket range (kNB when every remaining one fits), or blo when a single
// bucket holds more than the list.
template <int NT>
__device__ int bucket_batch(const uint32_t* Kp, int n, const BucketRange& br, BucketShared& bs, int blo) {
  const int t = (int)threadIdx.x;
  if (wave_id() == 0) {
    // the range: EXACT counts from blo in bucket order, 64 buckets a lane
    constexpr int PL = kNB / kWave;
    const int lane = lane_id();
    uint32_t c = 0;
    for (int i = 0; i < PL; ++i) {
      const int b = lane * PL + i;
      c += (b >= blo && bs.cls[bix(b)] == kBExact) ? bs.cnt[bix(b)] : 0u;
    }
    uint32_t ci = c;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const uint32_t o = __shfl_up(ci, d, kWave);
      if (lane >= d) ci += o;
    }
    uint32_t run = ci - c;
    int bhi = kNB;
    for (int i = 0; i < PL; ++i) {
      const int b = lane * PL + i;
      const bool ex = b >= blo && bs.cls[bix(b)] == kBExact;
      if (ex && run + bs.cnt[bix(b)] > (uint32_t)kBList && b < bhi) bhi = b;
      bs.off[bix(b)] = run;
      run += ex ? bs.cnt[bix(b)] : 0u;
    }
    bhi = (int)wave_min_u32((uint32_t)bhi);
    if (lane == 0) {
      bs.ctl[6] = (uint32_t)bhi;
      bs.nlist = 0u;
    }
  }
  __syncthreads();
  const int bhi = (int)bs.ctl[6];
  if (bhi == blo) return blo;
  for (int base = 0; base < n; base += NT * 8) {
    const int pos = base + t * 8;
    uint32_t k[8];
    bucket_keys8(Kp, pos, n, k);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (!br.in(k[i])) continue;
      const int b = br.of(k[i]);
      if (b >= blo && b < bhi && bs.cls[bix(b)] == kBExact) {
        const uint32_t slot = atomicAdd(&bs.nlist, 1u);  // < kBList: the range's counts fit
        bs.list[slot] = ((uint64_t)k[i] << 32) | (uint32_t)(pos + i);
      }
    }
  }
  __syncthreads();
  const int nl = (int)bs.nlist;
  int ns = 1;
  while (ns < nl) ns <<= 1;
  for (int i = nl + t; i < ns; i += NT) bs.list[i] = ~0ull;
  lds_barrier();
  // keys order the buckets, so the sorted list holds each bucket's elements
  // at its place (the exclusive count of EXACT buckets from blo before it)
  lds_bitonic_sort_u64<NT>(bs.list, ns);
  __syncthreads();
  return bhi;
}

// Why a walk stops (kWalkOk: the chain ended; kWalkMore: it reached the end
// of the batch's bucket range; the others decline the row).
enum : uint32_t { kWalkOk = 0, kWalkLeftBinade = 1, kWalkCutInPlain = 2, kWalkEndInPlain = 3, kWalkUnpredicted = 4,
                  kWalkPastRange = 5, kWalkMore = 6 };

// One walk over buckets [b_from, b_to) in key order by wave 0 (SUB: the
// draw), continuing from the running value v at position pos.  Positions
// [0, lim) take part; ADD stops at the first value > thr (thr < 0: never),
// SUB at the first value <= 0.  On kWalkOk: stop and the stopping element's
// position (pos), id and the value before it; or pos = lim.
template <bool SUB>
__device__ uint32_t bucket_walk(const BucketShared& bs, float& v, float& before, uint32_t& pos, uint32_t lim,
                                float thr, bool& stop, uint32_t& id_out, int b_from, int b_to) {
  const int lane = lane_id();
  stop = false;
  before = v;
  for (int b0 = b_from & ~(kWave - 1); b0 < b_to; b0 += kWave) {
    const int b = b0 + lane;  // < kNB
    const uint32_t cl = bs.cls[bix(b)];
    const int jb = bs.jg[bix(b)];
    const uint32_t sm = bs.sum[bix(b)], ct = bs.cnt[bix(b)], of = bs.off[bix(b)];
    int i = b0 < b_from ? b_from - b0 : 0;
    const int iend = min(kWave, b_to - b0);
    while (i < iend) {
      if (pos >= lim) return kWalkOk;
      const Grid g = grid_of(v);
      const bool live = lane >= i && lane < iend;
      const bool easy = live && (cl == kBEmpty || (cl == kBPlain && jb == g.j));
      const uint64_t hard = bal64(live && !easy);
      const int e = hard != 0ull ? __ffsll((long long)hard) - 1 : iend;
      const bool run = lane >= i && lane < e;
      const uint32_t add = wave_sum_sat(run && cl == kBPlain ? sm : 0u, kSat);
      const uint32_t pc = wave_sum_sat(run ? ct : 0u, 0x7fffffffu);
      if (e > i) {
        if (SUB) {
          if (add != 0u) {
            if (add >= g.N || g.N - add <= kGridBase) return kWalkLeftBinade;
            v = grid_value(g.N - add, g.j);
          }
        } else {
          if (add != 0u) {
            if (g.N + add >= kGridTop || g.N < kGridBase) return kWalkLeftBinade;
            v = grid_value(g.N + add, g.j);
          }
          if (thr >= 0.0f && v > thr) return kWalkCutInPlain;
        }
        pos += pc;
        if (pos > lim) return kWalkEndInPlain;
      }
      if (e >= iend) break;
      if (pos >= lim) return kWalkOk;
      if (readlane_u32(cl, e) != kBExact) return kWalkUnpredicted;  // NONE, or PLAIN on another grid
      const uint32_t o = readlane_u32(of, e);
      const uint32_t c = readlane_u32(ct, e);
      const int len = (int)min(c, lim - pos);
      int st;
      float bf;
      v = wave_seq_stop<SUB>(v, len, thr, st, bf, [&](int d) { return key_p((uint32_t)(bs.list[o + d] >> 32)); });
      if (st >= 0) {
        stop = true;
        before = bf;
        pos += (uint32_t)st;
        id_out = (uint32_t)bs.list[o + st];
        return kWalkOk;
      }
      pos += (uint32_t)len;
      i = e + 1;
    }
  }
  if (pos >= lim) return kWalkOk;
  return b_to < kNB ? kWalkMore : kWalkPastRange;
}

// A whole walk: PLAIN sums, then batches of EXACT buckets, each walked by
// wave 0 from where the last stopped.  Returns 0 or the decline reason; the
// results are broadcast through bs.ctl.
template <bool SUB, int NT>
__device__ uint32_t bucket_chain(const uint32_t* Kp, int n, const BucketRange& br, BucketShared& bs, float v0,
                                 uint32_t lim, float thr, float& v_out, float& before_out, uint32_t& pos_out,
                                 bool& stop_out, uint32_t& id_out, int row) {
  bucket_sums<NT>(Kp, n, br, bs);
  LLZ_STAMP(row, 29);
  float v = v0, before = v0;
  uint32_t pos = 0, id = 0xffffffffu, why = kWalkMore;
  bool stop = false;
  for (int blo = 0; why == kWalkMore;) {
    const int bhi = bucket_batch<NT>(Kp, n, br, bs, blo);
    if (bhi == blo) return 16u;  // one bucket holds more than the list
    if (blo == 0) LLZ_STAMP(row, 30);
    if (wave_id() == 0) {
      why = bucket_walk<SUB>(bs, v, before, pos, lim, thr, stop, id, blo, bhi);
      if (lane_id() == 0) {
        bs.ctl[0] = why;
        bs.ctl[1] = __float_as_uint(v);
        bs.ctl[2] = __float_as_uint(before);
        bs.ctl[3] = pos;
        bs.ctl[4] = stop ? 1u : 0u;
        bs.ctl[5] = id;
      }
    }
    __syncthreads();
    why = bs.ctl[0];
    v = __uint_as_float(bs.ctl[1]);
    before = __uint_as_float(bs.ctl[2]);
    pos = bs.ctl[3];
    stop = bs.ctl[4] != 0u;
    id = bs.ctl[5];
    __syncthreads();  // every thread has read ctl before a next batch writes it
    if (blo == 0) LLZ_STAMP(row, 31);
    blo = bhi;
  }
  v_out = v;
  before_out = before;
  pos_out = pos;
  stop_out = stop;
  id_out = id;
  return why;
}

}  // namespace llz
