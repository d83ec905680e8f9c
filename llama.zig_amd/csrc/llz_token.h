// llz_token.h -- the token of a row without its exact normaliser, for calls
// that ask for no probabilities and no row statistics (the reference's
// Sampler.sample returns the token alone, sampler.zig:26-28).
//
// Every decision of the chain after the normaliser S compares quantities
// that scale with 1/S (sampler.zig:90-168):
//   - the order (p desc, id asc) is the order of the terms e = exp((v-m)/T)
//     wherever two terms differ by more than 2^-21 relative (then their
//     quotients by any S round to different floats) or are equal;
//   - min-p compares RN(e / S) with RN(RN(1 / S) min_p): a term above
//     min_p (1 + 2^-22) passes and one below min_p (1 - 2^-22) fails,
//     whatever S (three roundings of 2^-24 each);
//   - the draw: r_q = RN(r_{q-1} - p_q) from RN(u * total) stops at the
//     first r_q <= 0; with E the sum of the kept terms and C_q the sum of the
//     first q+1, S r_q differs from u E - C_q by at most (3K + 7) 2^-24 E
//     (K kept terms: the sums' and quotients' roundings), so a row whose
//     u E - C_q stay clear of that band stops where the sign of u E - C_q
//     first turns, whatever S;
//   - top-p compares the running sum, which lies within (2q + 4) 2^-24 of
//     C_q / S, with top_p: that needs S itself.  The reference's S is the
//     sequential f32 sum of n positive terms, within (n - 1) 2^-24 / (1 - (n -
//     1) 2^-24) of the real sum (the recursive-summation bound), or within
//     about 2^-24 sum_j e_j (n - j + 1) / S, the same bound by where the mass
//     lies (an estimate of it comes with S's), which phase L's estimates
//     give to 2^-14 (2^-14 + est_xe on soft-capped rows); a top-p decision
//     that holds at both ends of that interval holds at S.
// A row whose decisions all hold is finished here, bit-exact; any other row
// continues with the exact phases.
#pragma once

#include "llz_internal.h"
#include "llz_norm.h"
#include "llz_wg.h"

namespace llz {

constexpr int kTokCap = 512;  // candidates of a token-only row at most

// Rank sort of c <= kTokCap distinct keys (e desc as ~bits, id asc) for
// wave 0: wave w counts, for every key, the keys of its eighth of the list
// below it (part[w][i], at most kTokCap / 8 = 64: one byte, no clearing
// needed); after one barrier wave 0 adds the eight counts and places each
// key.  Only wave 0 reads `out` (in LDS order after its own writes).
__device__ __forceinline__ void token_sort(const uint64_t* in, uint64_t* out, uint8_t* part, int c) {
  static_assert(kTokCap / (kNT / kWave) <= 255, "partial ranks fit a byte");
  constexpr int NW = kNT / kWave;
  const int lane = lane_id(), w = wave_id();
  const int j0 = (w * c) / NW, j1 = ((w + 1) * c) / NW;
  for (int i = lane; i < c; i += kWave) {
    const uint64_t ki = in[i];
    uint32_t r = 0;
    for (int j = j0; j < j1; ++j) r += in[j] < ki ? 1u : 0u;
    part[w * kTokCap + i] = (uint8_t)r;
  }
  lds_barrier();
  if (w == 0) {
    for (int i = lane; i < c; i += kWave) {
      uint32_t r = 0;
#pragma unroll
      for (int v = 0; v < NW; ++v) r += part[v * kTokCap + i];
      out[r] = in[i];
    }
    __builtin_amdgcn_wave_barrier();
  }
}

__device__ __forceinline__ double readlane_f64(double v, int l) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = readlane_u32((uint32_t)b, l), hi = readlane_u32((uint32_t)(b >> 32), l);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// DPP move of a double (both halves), lanes the control leaves out get 0.
template <int CTRL, int RM, int BM, bool BC>
__device__ __forceinline__ double dpp_f64(double x) {
  const uint64_t b = (uint64_t)__double_as_longlong(x);
  const uint32_t lo = dpp_u32<CTRL, RM, BM, BC>(0u, (uint32_t)b);
  const uint32_t hi = dpp_u32<CTRL, RM, BM, BC>(0u, (uint32_t)(b >> 32));
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Inclusive prefix sum within a wave (the DPP pattern of wave_incl_scan_op).
__device__ __forceinline__ double wave_incl_scan_f64(double x) {
  double s = x;
  s = s + dpp_f64<0x111, 0xf, 0xf, true>(x);
  s = s + dpp_f64<0x112, 0xf, 0xf, true>(x);
  s = s + dpp_f64<0x113, 0xf, 0xf, true>(x);
  s = s + dpp_f64<0x114, 0xf, 0xe, false>(s);
  s = s + dpp_f64<0x118, 0xf, 0xc, false>(s);
  s = s + dpp_f64<0x142, 0xa, 0xf, false>(s);
  s = s + dpp_f64<0x143, 0xc, 0xf, false>(s);
  return s;
}

// Typical-p on the token path (sampler.zig:128-154).  The entropy is that
// of the row's terms e_i <= 1 (their real sum S):
//   H* = ln S - (1/S) sum_i e_i ln e_i = ln 2 (log2 S - Y / S),
//   Y = sum_i e_i log2 e_i <= 0.
// Each wave sums q (log2 q + aw) over its estimates (q R_w = e (1 + d),
// |d| <= de = 2^-14 + est_xe, R_w = exp2(aw)), with the hardware log2 (within
// 2^-18 max(1, |log2 q|) of log2 q) and the magnitudes of those terms (A_w).
// Per element, with the computed term's roundings (one for the sum in the
// brackets, one for the product, about 260 for the lane's and the wave's
// sums), the distance to e log2 e is within de e |log2 e| + e (1.5 de +
// 2^-17.9 (1 + |log2 e| + |aw|)) + 2^-15 |term|, so |Y - sum_w R_w X_w| <=
// sum_w R_w (A_w (de + 2^-14.47) + Q_w (1.5 de + 2^-14.47 (1 + |aw|)))
// (Q_w: the wave's sum of q), widened by 2^-8 of itself for the use of the
// estimates in place of the terms; terms with q < 2^-100 are left out (far
// below 2^-60 in all).  S lies within s_est / (1 +- de).
__device__ __forceinline__ void entropy_star(const RowParams& P, const float* tx, const float* txa, const float* qsum,
                                          const float* cwv, int nw, int G, float m, float s_est, double* lo,
                                          double* hi) {
  const double de = 0x1p-14 + (double)P.est_xe;
  double X = 0.0, B = 0.0;
  for (int i = 0; i < nw; ++i) {
    if (G > i) {
      const float awi = fmaf(m, -P.l2e_t, cwv[i]);
      const double ri = (double)__builtin_amdgcn_exp2f(awi);
      X += ri * (double)tx[i];
      B += ri * ((double)txa[i] * (de + 0x1.7p-15) + (double)qsum[i] * (1.5 * de + 0x1.7p-15 * (1.0 + fabs((double)awi))));
    }
  }
  const double EY = B * (1.0 + 0x1p-8) + fabs(X) * 0x1p-40 + 0x1p-60;
  const double Smin = (double)s_est / (1.0 + de) * (1.0 - 0x1p-50), Smax = (double)s_est / (1.0 - de) * (1.0 + 0x1p-50);
  const double Nlo = -X - EY, Nhi = -X + EY;  // -Y lies in [Nlo, Nhi]
  const double Alo = log2(Smin) + (Nlo >= 0.0 ? Nlo / Smax : Nlo / Smin);
  const double Ahi = log2(Smax) + (Nhi >= 0.0 ? Nhi / Smin : Nhi / Smax);
  const double ln2 = 0.69314718055994530942;
  *lo = ln2 * Alo - 0x1p-40 * (fabs(Alo) + 1.0);
  *hi = ln2 * Ahi + 0x1p-40 * (fabs(Ahi) + 1.0);
  if (!(Smin > 0.0) || !(*lo <= *hi) || !(fabs(*hi) < 1.0e30)) {
    *lo = 0.0;
    *hi = -1.0;
  }
}

// Wave 0: the chain's decisions (sampler.zig:100-168) for a token-only row
// from its candidates srt[0, c), sorted (e desc, id asc) -- every term e >=
// theta, all of them exact -- and the estimate s_est of the normaliser
// (w_est: of sum_j e_j (n - j), an upper bound's estimate; 0: unknown), and
// for typical-p the interval [hs_lo, hs_hi] of the row's entropy H*
// (entropy_star; empty: unknown, and then only rows that keep nothing
// before typical-p are decided).  Writes the token, the draw flag, the kept
// count and ids; sets *tfail instead when a decision does not hold over the
// intervals.
// TYP false leaves typical-p's decisions out of the code (its rows are then
// decided only when they keep nothing before typical-p).
// Out of line; the launch's arguments come through the kernel's argument
// segment (as the other out-of-line paths take them).
template <bool TYP>
__device__ __forceinline__ void token_select(const KArgs* A, int row, const uint64_t* srt, int c, float s_est,
                                          float w_est, double hs_lo, double hs_hi, float u, float theta,
                                          uint32_t* tfail) {
  const RowParams& P = A->P;
  const RowPtrs& Q = A->Q;
  const int lane = lane_id();
  const int n = P.n;
  // the first kWave + 1 keys, read once: lane q holds keys q and q + 1
  // (lists of at most kWave, the common case, read nothing more)
  const uint64_t k0 = lane < c ? srt[lane] : ~0ull;
  const uint64_t k1 = lane + 1 < c ? srt[lane + 1] : ~0ull;
  auto e_of = [](uint64_t k) { return __uint_as_float(~(uint32_t)(k >> 32)); };
  auto e_at = [&](int q) { return q < kWave ? e_of(k0) : e_of(srt[q]); };  // q: this lane's own position
  auto e_next = [&](int q) { return q < kWave ? e_of(k1) : e_of(srt[q + 1]); };
  auto id_at = [&](int q) { return (uint32_t)srt[q]; };
  bool ok = c >= 1;
  // certified prefix M: list terms clear of every term outside the list
  // (< theta); min-p: p < RN(RN(1/S) min_p) exactly for the terms below
  // mp_lo, never for those above mp_hi, and the terms past M lie below
  // theta (1 + 2^-21) < min_p (1 - 2^-21)
  const float th_hi = theta * (1.0f + 0x1p-21f);
  const bool mp = P.min_p > 0.0f;
  const float mp_hi = P.min_p * (1.0f + 0x1p-22f), mp_lo = P.min_p * (1.0f - 0x1p-22f);
  int M = 0, Km = 0;
  for (int b = 0; b < c; b += kWave) {
    const int q = b + lane;
    const float e = q < c ? e_at(q) : 0.0f;
    const bool inM = q < c && (theta == 0.0f || e > th_hi);
    M += __popcll(bal64(inM));
    Km += __popcll(bal64(inM && e > mp_hi));
    if (mp && bal64(inM && !(e > mp_hi) && !(e < mp_lo)) != 0ull) ok = false;
  }
  // a list collected again above theta > tok_theta (top-k) may leave out
  // terms that pass min-p: when every certified term passes it, min-p's
  // count is unknown beyond the list (the kept prefix then ends at top-k
  // inside it, or at top-p's cut)
  if (!mp || (theta > P.tok_theta && Km == M)) Km = n;
  LLZ_STAMP(row, 35);
  const int Kk = (P.top_k > 0 && P.top_k < (uint32_t)n) ? (int)P.top_k : n;
  const int L = min(Kk, Km);
  // a kept prefix that may reach past the certified prefix (no min-p, and
  // no top-k inside it) is decided only by a top-p cut inside the prefix:
  // the terms outside the list come after every position below M, and
  // top-p, applied before min-p, drops each of them once it has cut
  const bool open_end = L > M;
  const int Lc = open_end ? M : L;
  // the interval of the reference's normaliser
  double rs = P.tok_rs;  // g / (1 - g), g = (n - 1) 2^-24 (host)
  // The same bound by where the mass lies (w_est > 0): the computed partial
  // sums of positive terms satisfy S^_i <= S_i (1 + gamma_i), so |S^ - S| <=
  // u / (1 - u) sum_{i>=2} S^_i <= u / (1 - u) (1 + gamma_n) sum_i S_i, and
  // sum_i S_i = sum_j e_j (n - j + 1) (j 1-based: e_j lies in the partial
  // sums from the j-th on) <= W, estimated by w_est as s_est estimates S,
  // so W / S <= (w_est / s_est) (1 + e) / (1 - e) <= (w_est / s_est) (1 +
  // 2^-9) (e = 2^-14 + est_xe <= 2^-10.8).  With the row's mass spread
  // evenly this halves the interval; with it near the row's end, far more.
  // (tok_rwk = u / (1 - u) (1 + gamma_n) (1 + 2^-9) from the host, 0 when
  // gamma_n >= 1/2; the ratio from above: a correctly rounded f32 quotient
  // widened by its half ulp)
  if (w_est > 0.0f && P.tok_rwk > 0.0) {
    const double rw = P.tok_rwk * ((double)(w_est / s_est) * (1.0 + 0x1p-23));
    if (rw < rs) rs = rw;
  }
  // the estimate's own error e; S^ in s_est [(1 - rs)(1 - e), (1 + rs)(1 + e)]
  const double e_est = 0x1p-14 + (double)P.est_xe;  // est_xe: soft-capped rows' estimates
  const double gr = rs + e_est + rs * e_est;
  const double S_lo = (double)s_est * (1.0 - gr), S_hi = (double)s_est * (1.0 + gr);
  if (!(S_lo > 0.0) || !(S_hi < 1.0e300)) ok = false;
  // 1/S at the interval's ends, rounded outwards (one rounding of 2^-53 each)
  const double iS_hi = (1.0 / S_hi) * (1.0 - 0x1p-50), iS_lo = (1.0 / S_lo) * (1.0 + 0x1p-50);
  const bool topp = P.top_p > 0.0f && P.top_p < 1.0f;
  // one pass over positions [0, Lc): the running sums C_q of the terms
  // (double), top-p's cut (sampler.zig:111-118), and the order: adjacent terms
  // up to max(L, 1) equal (then ordered by id) or apart by more than 2^-21
  const int pe = min(max(L, 1), M - 1);
  const int span = max(Lc, pe);
  double carry = 0.0, C0 = 0.0;  // C0: lane q's C_q for q < 64
  int cut = -1;
  for (int b = 0; b < span && ok && cut < 0; b += kWave) {
    const int q = b + lane;
    const float e = q < c ? e_at(q) : 0.0f;
    const double C = carry + wave_incl_scan_f64(q < Lc ? (double)e : 0.0);
    if (b == 0) C0 = C;
    if (topp) {
      const double rel = (2.0 * q + 4.0) * 0x1p-24;
      const bool lo_over = q < Lc && C * iS_hi * (1.0 - rel) > (double)P.top_p;
      const bool hi_over = q < Lc && C * iS_lo * (1.0 + rel) > (double)P.top_p;
      const uint64_t mh = bal64(hi_over);
      if (mh != 0ull) {
        const int fq = __ffsll((long long)mh) - 1;
        if ((bal64(lo_over) >> fq) & 1ull)
          cut = b + fq;
        else
          ok = false;
      }
    }
    bool unc = false;
    if (q < pe) {
      const float eb = e_next(q);
      unc = e != eb && !(e > eb * (1.0f + 0x1p-21f));
    }
    if (bal64(unc) != 0ull) ok = false;
    carry = readlane_f64(C, kWave - 1);
  }
  if (open_end && cut < 0) ok = false;  // the kept prefix may reach past the list
  const int K = cut >= 0 ? min(L, cut) : L;
  LLZ_STAMP(row, 36);
  // C_j = e_0 + ... + e_j for j < K (exact in double: at most kTokCap f32
  // terms in [theta, 1], theta >= 2^-11)
  auto prefix = [&](int j) -> double {
    if (j < kWave) return readlane_f64(C0, j);
    double acc = 0.0;
    for (int b = 0; b <= j; b += kWave) {
      const int q = b + lane;
      acc += readlane_f64(wave_incl_scan_f64(q <= j ? (double)e_at(q) : 0.0), kWave - 1);
    }
    return acc;
  };
  // typical-p (sampler.zig:128-154) over the kept positions [0, K); the
  // positions kept after it are [a, b)
  int a = 0, b = K;
  if (!TYP && K > 0 && P.typical_p > 0.0f && P.typical_p < 1.0f) ok = false;
  // When the running sum of all K kept terms stays at most typical_p
  // whatever S (the largest of the running sums in any order), typical-p
  // drops nothing, and neither the entropy nor the order matters
  bool typ_cut = false;
  if constexpr (TYP) {
    if (ok && K > 0 && P.typical_p > 0.0f && P.typical_p < 1.0f)
      typ_cut = !(prefix(K - 1) * iS_lo * (1.0 + (2.0 * K + 4.0) * 0x1p-24) <= (double)P.typical_p);
  }
  if constexpr (TYP) if (typ_cut) {
    // The reference's entropy H^ (sampler.zig:129-132): the sequential sum of
    // t_i = -RN(p_i logf(p_i)), p_i = RN(e_i / S^).  With pi_i = e_i / S^ and
    // h_i = -pi_i ln pi_i, |t_i - h_i| <= 2^-21.9 h_i + 2^-23.9 pi_i (p's,
    // logf's and the product's roundings); sum_i h_i = c (H* - ln c), c = S /
    // S^ in [1 / (1 + rs), 1 / (1 - rs)]; the sum's roundings add
    // gamma_{n-1} of it (all t_i >= 0).
    bool known = hs_lo <= hs_hi;
    const double c_lo = 1.0 / (1.0 + rs), c_hi = 1.0 / (1.0 - rs);
    const double kap = c_hi * fmax(fabs(log(c_lo)), fabs(log(c_hi)));
    const double sh_lo = fmin(c_lo * hs_lo, c_hi * hs_lo) - kap, sh_hi = fmax(c_lo * hs_hi, c_hi * hs_hi) + kap;
    const double t_lo = sh_lo - fabs(sh_lo) * 0x1.2p-22 - 0x1.2p-24 * c_hi - 0x1p-100;
    const double t_hi = sh_hi + fabs(sh_hi) * 0x1.2p-22 + 0x1.2p-24 * c_hi + 0x1p-100;
    const double gn1 = (double)(n - 1) * 0x1p-24;
    const double gH = gn1 / (1.0 - gn1) * (1.0 + 0x1p-40);
    const double H_lo = t_lo - fabs(t_lo) * gH, H_hi = t_hi + fabs(t_hi) * gH;
    known = known && gn1 < 0.5;
    // surprises s_j = -logf(p_j) (sampler.zig:140): -ln p_j lies within
    // ln S^ - ln e_j +- 1.01 2^-24, logf within 2^-23 of ln; s_j grows with j
    const double u24 = 0x1p-24;
    const double le0 = log((double)e_of(srt[0])), leK = log((double)e_of(srt[K - 1]));
    const double lSlo = log(S_lo), lShi = log(S_hi);
    const double s0_lo = (lSlo - le0 - 1.01 * u24) * (1.0 - 0x1p-23) - 0x1p-45 * (fabs(lSlo) + fabs(le0) + 1.0);
    const double sK_hi = (lShi - leK + 1.01 * u24) * (1.0 + 0x1p-23) + 0x1p-45 * (fabs(lShi) + fabs(leK) + 1.0);
    // every kept surprise below the entropy (dev_j = H^ - s_j: the typical
    // order is positions K-1 .. 0) or every one above it (dev_j = s_j - H^:
    // positions 0 .. K-1), whatever S^ and H^ in their intervals
    const bool below = known && sK_hi < H_lo;
    const bool above = known && s0_lo > H_hi;
    if (!below && !above) ok = false;
    // no two kept devs round to one float (a tie would take the lower id
    // first): adjacent terms apart by mu relative put their surprises more
    // than 2^-21 max dev apart
    const double mu = 0x1p-20 * (fmax(H_hi, sK_hi) + sK_hi + 1.0);
    for (int bb = 0; bb < K - 1 && ok; bb += kWave) {
      const int q = bb + lane;
      const bool bad = q < K - 1 && !((double)e_at(q) > (double)e_next(q) * (1.0 + mu));
      if (bal64(bad) != 0ull) ok = false;
    }
    // the cut (sampler.zig:148-153): the running sum of p over the kept
    // terms in the typical order, within (2r + 4) 2^-24 of the terms' sum /
    // S^ after r of them, against typical_p; the term that takes it over and
    // every later one are dropped
    const double tp = (double)P.typical_p;
    if (ok && above) {
      double carry = 0.0;
      int bc = -1;
      for (int bb = 0; bb < K && ok && bc < 0; bb += kWave) {
        const int q = bb + lane;
        const double C = carry + wave_incl_scan_f64(q < K ? (double)e_at(q) : 0.0);
        const double rel = (2.0 * q + 4.0) * u24;
        const bool lo_over = q < K && C * iS_hi * (1.0 - rel) > tp;
        const bool hi_over = q < K && C * iS_lo * (1.0 + rel) > tp;
        const uint64_t mh = bal64(hi_over);
        if (mh != 0ull) {
          const int fq = __ffsll((long long)mh) - 1;
          if ((bal64(lo_over) >> fq) & 1ull)
            bc = bb + fq;
          else
            ok = false;
        }
        carry = readlane_f64(C, kWave - 1);
      }
      b = bc >= 0 ? bc : K;
    } else if (ok) {
      // positions K-1 .. j hold D_j = E_K - C_j + e_j; the last position
      // whose sum may exceed typical_p is where the cut falls
      const double EK = prefix(K - 1);
      double carry = 0.0;
      int jh = -1;
      bool jlo = false;
      for (int bb = 0; bb < K; bb += kWave) {
        const int q = bb + lane;
        const double eq = q < K ? (double)e_at(q) : 0.0;
        const double C = carry + wave_incl_scan_f64(eq);
        const double D = EK - C + eq;
        const double rel = (2.0 * (K - q) + 4.0) * u24;
        const bool hi_over = q < K && D * iS_lo * (1.0 + rel) > tp;
        const bool lo_over = q < K && D * iS_hi * (1.0 - rel) > tp;
        const uint64_t mh = bal64(hi_over);
        if (mh != 0ull) {
          const int fq = 63 - __clzll((long long)mh);
          jh = bb + fq;
          jlo = ((bal64(lo_over) >> fq) & 1ull) != 0ull;
        }
        carry = readlane_f64(C, kWave - 1);
      }
      if (jh >= 0 && !jlo) ok = false;
      a = jh + 1;
    }
  }
  const int Kp = b - a;  // the kept count
  uint32_t token = c >= 1 ? readlane_u32((uint32_t)k0, 0) : 0u, consumed = 0;  // indices[0]
  if constexpr (TYP) {
    if (ok && Kp > 0) {
      // total and draw (sampler.zig:156-168) over positions [a, b): E = C_{b-1}
      // - C_{a-1}; the draw stops at the first q with u E - (C_q - C_{a-1})
      // below -margin (none of them within it)
      const double Ca = a > 0 ? prefix(a - 1) : 0.0;
      const double E = prefix(b - 1) - Ca;
      const double Au = (double)u * E;
      const double margin = (4.0 * Kp + 16.0) * 0x1p-24 * E;
      int st = -1;
      double dcarry = 0.0;
      for (int bb = 0; bb < b && st < 0 && ok; bb += kWave) {
        const int q = bb + lane;
        const double C = bb == 0 ? C0 : dcarry + wave_incl_scan_f64(q < K ? (double)e_at(q) : 0.0);
        const double dq = Au - (C - Ca);
        const bool in = q >= a && q < b;
        const bool unc = in && fabs(dq) <= margin;
        const bool stp = in && dq < -margin;
        const uint64_t mk = bal64(unc || stp);
        if (mk != 0ull) {
          const int fq = __ffsll((long long)mk) - 1;
          if ((bal64(unc) >> fq) & 1ull)
            ok = false;
          else
            st = bb + fq;
        }
        dcarry = readlane_f64(C, kWave - 1);
      }
      consumed = 1;
      if (st >= 0) token = st < kWave ? readlane_u32((uint32_t)k0, st) : id_at(st);
    }
  } else if (ok && K > 0) {
    // total and draw (sampler.zig:156-168): E = C_{K-1}; the draw stops at
    // the first q with u E - C_q below -margin (none of them within it)
    double E;
    if (K <= kWave) {
      E = readlane_f64(C0, K - 1);
    } else {
      E = 0.0;
      for (int bb = 0; bb < K; bb += kWave) {
        const int q = bb + lane;
        E += readlane_f64(wave_incl_scan_f64(q < K ? (double)e_at(q) : 0.0), kWave - 1);
      }
    }
    const double Au = (double)u * E;
    const double margin = (4.0 * K + 16.0) * 0x1p-24 * E;
    int st = -1;
    double dcarry = 0.0;
    for (int bb = 0; bb < K && st < 0 && ok; bb += kWave) {
      const int q = bb + lane;
      const double C = bb == 0 ? C0 : dcarry + wave_incl_scan_f64(q < K ? (double)e_at(q) : 0.0);
      const double dq = Au - C;
      const bool unc = q < K && fabs(dq) <= margin;
      const bool stp = q < K && dq < -margin;
      const uint64_t mk = bal64(unc || stp);
      if (mk != 0ull) {
        const int fq = __ffsll((long long)mk) - 1;
        if ((bal64(unc) >> fq) & 1ull)
          ok = false;
        else
          st = bb + fq;
      }
      dcarry = readlane_f64(C, kWave - 1);
    }
    consumed = 1;
    if (st >= 0) token = st < kWave ? readlane_u32((uint32_t)k0, st) : id_at(st);
  }
  LLZ_STAMP(row, 37);
  if (!ok) {
    if (lane == 0) *tfail = 1u;
    return;
  }
  if (Q.kept_ids)
    for (int q = lane; q < Kp && q < P.kept_cap; q += kWave)
      Q.kept_ids[(int64_t)row * P.kept_cap + q] = (a == 0 && q < kWave) ? (uint32_t)k0 : id_at(a + q);
  if (lane == 0) {
    Q.tokens[row] = token;
    if (Q.consumed) Q.consumed[row] = (uint8_t)consumed;
    if (Q.kept_count) Q.kept_count[row] = (uint32_t)Kp;
    if (Q.status) Q.status[row] = kPathTokenOnly;
  }
}

}  // namespace llz
