// llz_kernels.hip -- MI355X (gfx950) kernels for llama.zig's sampling chain.
//
// Pipeline per call (rows are independent; each row is one workgroup in the
// sampling kernel):
//   k_penalty  (optional) penalised copy of the rows      sampler.zig:54-75
//   k_rowmax   partial maxima, many workgroups per row     sampler.zig:80-81
//   k_sample   one 1024-thread workgroup per row:
//                exact sequential normaliser + candidates  sampler.zig:83-90
//                candidate sort by (p desc, id asc)         sampler.zig:92-100
//                top-k / top-p / min-p                      sampler.zig:106-126
//                typical-p (entropy pass, dev sort)         sampler.zig:128-154
//                total and the draw                         sampler.zig:156-168
//              with a full-row radix-sort fallback for rows whose kept set
//              does not fit the candidate list.
//   k_argmax   greedy rows (temperature <= 0)             sampler.zig:31-41,50
#include <hip/hip_runtime.h>

#include "llz_accum.h"
#include "llz_internal.h"
#include "llz_math.h"
#include "llz_wg.h"

namespace llz {

constexpr int kNT = 1024;          // threads of the per-row workgroup
constexpr int kV = 4;              // logits per thread per streaming tile
constexpr int kTile = kNT * kV;    // 4096 logits per tile
constexpr int kCap = kCandCap;     // candidate list capacity (power of two)
constexpr int kMaxNT = 256;        // threads of the k_rowmax / k_penalty workgroups
constexpr int kMaxPerThread = 16;  // logits per thread in k_rowmax
constexpr float kInf = __builtin_inff();

// ---------------------------------------------------------------------------
// small helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_fmax(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}

template <int NT>
__device__ __forceinline__ float wg_fmax(float v, WgScratch<NT>& sh, int& bank) {
  v = wave_fmax(v);
  if (lane_id() == 0) sh.red[bank][wave_id()] = __float_as_uint(v);
  __syncthreads();
  float r = __uint_as_float(sh.red[bank][0]);
#pragma unroll
  for (int w = 1; w < WgScratch<NT>::W; ++w) r = fmaxf(r, __uint_as_float(sh.red[bank][w]));
  bank ^= 1;
  return r;
}

// (value, index) ordering of sampleArgmax (sampler.zig:31-41): larger value
// wins, equal values keep the lower index, NaN never wins.
__device__ __forceinline__ bool amax_better(float v, uint32_t i, float bv, uint32_t bi) {
  if (v != v) return false;
  if (bv != bv) return true;
  return v > bv || (v == bv && i < bi);
}

// sampleArgmax over one row with the whole workgroup.  A NaN at index 0
// is never replaced by the reference's loop, so the answer is then 0.
template <int NT>
__device__ uint32_t wg_argmax_row(const float* x, int n, WgScratch<NT>& sh, int& bank) {
  const int t = (int)threadIdx.x;
  float bv = __builtin_nanf("");
  uint32_t bi = 0xffffffffu;
  for (int i = t; i < n; i += NT) {
    const float v = x[i];
    if (amax_better(v, (uint32_t)i, bv, bi)) { bv = v; bi = (uint32_t)i; }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(bv, m, kWave);
    const uint32_t oi = __shfl_xor(bi, m, kWave);
    if (amax_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  if (lane_id() == 0) {
    sh.red[bank][wave_id()] = bi;
    sh.red[bank ^ 1][wave_id()] = __float_as_uint(bv);
  }
  __syncthreads();
  float rv = __builtin_nanf("");
  uint32_t ri = 0xffffffffu;
  for (int w = 0; w < WgScratch<NT>::W; ++w) {
    const float v = __uint_as_float(sh.red[bank ^ 1][w]);
    const uint32_t i = sh.red[bank][w];
    if (amax_better(v, i, rv, ri)) { rv = v; ri = i; }
  }
  __syncthreads();  // both banks were used
  const float x0 = x[0];
  if (x0 != x0 || ri == 0xffffffffu) ri = 0;
  return ri;
}

// Load kV consecutive logits starting at pos (positions >= n read as 0).
__device__ __forceinline__ void load4(const float* row, int pos, int n, bool vec, float (&v)[kV]) {
  if (vec && pos + kV <= n) {
    const float4 q = *reinterpret_cast<const float4*>(row + pos);
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  } else {
#pragma unroll
    for (int k = 0; k < kV; ++k) v[k] = pos + k < n ? row[pos + k] : 0.0f;
  }
}

// e_i = exp((v_i - max) / T) as sampler.zig:85 evaluates it.
__device__ __forceinline__ float row_exp(float v, float m, float T, bool t_is_one) {
  float x = v - m;
  if (!t_is_one) x = x / T;  // x / 1.0f == x exactly, so the divide is skipped
  return exp_f32(x);
}

// ---------------------------------------------------------------------------
// k_penalty: penalised copy (sampler.zig:54-75).  Each index is penalised at
// most once even when it repeats in the window (the reference breaks out of
// the window scan at the first match).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kMaxNT) void k_penalty(const float* __restrict__ logits, int64_t stride,
                                                    int n, const uint32_t* __restrict__ prev,
                                                    int n_prev, int64_t prev_stride, int window,
                                                    float penalty, float* __restrict__ out) {
  const int row = blockIdx.y;
  const int seg0 = blockIdx.x * (kMaxNT * kMaxPerThread);
  const int seg1 = min(n, seg0 + kMaxNT * kMaxPerThread);
  const float* x = logits + (int64_t)row * stride;
  float* y = out + (int64_t)row * n;
  for (int i = seg0 + (int)threadIdx.x; i < seg1; i += kMaxNT) y[i] = x[i];
  __syncthreads();
  const uint32_t* pv = prev + (int64_t)row * prev_stride;
  const int w = min(n_prev, window);
  const int start = n_prev - w;
  for (int a = start + (int)threadIdx.x; a < n_prev; a += kMaxNT) {
    const uint32_t tok = pv[a];
    if (tok >= (uint32_t)seg0 && tok < (uint32_t)seg1) {
      bool first = true;
      for (int b = start; b < a; ++b) first = first && (pv[b] != tok);
      if (first) {
        const float v = x[tok];
        y[tok] = v > 0.0f ? v / penalty : v * penalty;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// k_rowmax: partial row maxima with @max's NaN-ignoring semantics.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kMaxNT) void k_rowmax(const float* __restrict__ logits, int64_t stride,
                                                   int n, int nparts, int vec,
                                                   float* __restrict__ part) {
  const int row = blockIdx.y;
  const int seg0 = blockIdx.x * (kMaxNT * kMaxPerThread);
  const float* x = logits + (int64_t)row * stride;
  float m = -kInf;
  bool seen_num = false;
  if (vec) {
    float4 q[kMaxPerThread / 4];
#pragma unroll
    for (int c = 0; c < kMaxPerThread / 4; ++c) {
      const int pos = seg0 + (c * kMaxNT + (int)threadIdx.x) * 4;
      q[c] = pos + 4 <= n ? *reinterpret_cast<const float4*>(x + pos)
                          : make_float4(__builtin_nanf(""), __builtin_nanf(""),
                                        __builtin_nanf(""), __builtin_nanf(""));
      if (pos + 4 > n) {
        if (pos + 0 < n) q[c].x = x[pos + 0];
        if (pos + 1 < n) q[c].y = x[pos + 1];
        if (pos + 2 < n) q[c].z = x[pos + 2];
      }
    }
#pragma unroll
    for (int c = 0; c < kMaxPerThread / 4; ++c) {
      m = fmaxf(m, q[c].x); m = fmaxf(m, q[c].y); m = fmaxf(m, q[c].z); m = fmaxf(m, q[c].w);
    }
    seen_num = true;
  } else {
    for (int k = 0; k < kMaxPerThread; ++k) {
      const int pos = seg0 + k * kMaxNT + (int)threadIdx.x;
      if (pos < n) m = fmaxf(m, x[pos]);
    }
    seen_num = true;
  }
  (void)seen_num;
  // all-NaN segments give -inf here; the reference's fold would give NaN
  // only when every logit of the row is NaN (handled in k_sample).
  __shared__ float red[kMaxNT / kWave];
  m = wave_fmax(m);
  if (lane_id() == 0) red[wave_id()] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = red[0];
    for (int w = 1; w < kMaxNT / kWave; ++w) r = fmaxf(r, red[w]);
    part[(int64_t)row * nparts + blockIdx.x] = r;
  }
}

// ---------------------------------------------------------------------------
// k_argmax: one workgroup per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kNT) void k_argmax(const float* __restrict__ logits, int64_t stride,
                                                int n, uint32_t* __restrict__ tokens,
                                                uint8_t* __restrict__ consumed,
                                                uint32_t* __restrict__ kept_count) {
  __shared__ WgScratch<kNT> sh;
  int bank = 0;
  const int row = blockIdx.x;
  const uint32_t tok = wg_argmax_row<kNT>(logits + (int64_t)row * stride, n, sh, bank);
  if (threadIdx.x == 0) {
    tokens[row] = tok;
    if (consumed) consumed[row] = 0;
    if (kept_count) kept_count[row] = 0;
  }
}

// ---------------------------------------------------------------------------
// k_sample
// ---------------------------------------------------------------------------
struct SampleShared {
  WgScratch<kNT> wg;
  uint32_t cand_count;
  uint32_t misc[4];
  uint64_t cand[kCap];      // (e bits, id) while collecting, then (~p bits, id) sorted
  uint64_t aux[kCap];       // (dev bits, id) for typical-p
  uint32_t aux_pos[kCap];   // p-order position carried through the dev sort
  uint8_t keep[kCap];       // final keep flag per p-order position
  RadixScratch radix;
};

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
      __syncthreads();
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
    list_accumulate<kNT, 2, false>(0.0f, lim, P.top_p, st, [&](int q) { return L.p(q); }, sh.wg, bank);
    if (st >= 0) Kp = st;
    else if (bound > M) return -1;  // the cut may lie beyond the certified prefix
  }
  (void)km_known;  // an unknown Km >= M only matters if the result exceeds M
  const int K = min(Kk, min(Kp, Km));
  return K > M ? -1 : K;
}

// Entropy sum over the whole row in index order (sampler.zig:129-132).
__device__ float entropy_pass(const float* xr, int n, float m, float S, const RowParams& P,
                              SampleShared& sh, int& bank) {
  const bool t1 = (P.flags & kFlagTIsOne) != 0;
  const bool vec = (P.flags & kFlagVecSrc) != 0;
  float H = 0.0f;
  const int t = (int)threadIdx.x;
  for (int base = 0; base < n; base += kTile) {
    float v[kV], term[kV];
    load4(xr, base + t * kV, n, vec, v);
#pragma unroll
    for (int k = 0; k < kV; ++k) {
      const float p = row_exp(v[k], m, P.temperature, t1) / S;
      // entropy -= p * log(p) for p > 0; the term enters negated (exact)
      term[k] = p > 0.0f ? -(p * log_f32(p)) : -0.0f;
    }
    int st;
    H = tile_accumulate<kNT, kV, false>(H, term, min(kTile, n - base), -1.0f, st, sh.wg, bank);
  }
  return H;
}

// Total and draw over p-order positions [0, K) whose keep flag is set
// (sampler.zig:156-168).  keep(q) -> bool.
template <typename List, typename Keep>
__device__ void total_and_draw(const List& L, int K, Keep keep, float u, float& total,
                               uint32_t& token, uint32_t& consumed, SampleShared& sh, int& bank) {
  int st;
  total = list_accumulate<kNT, 2, false>(
      0.0f, K, -1.0f, st, [&](int q) { return keep(q) ? L.p(q) : -0.0f; }, sh.wg, bank);
  const uint32_t tok0 = L.id(0);
  if (total <= 0.0f) {
    token = tok0;
    consumed = 0;
    return;
  }
  consumed = 1;
  const float r0 = u * total;
  list_accumulate<kNT, 2, true>(r0, K, -1.0f, st, [&](int q) { return keep(q) ? L.p(q) : -0.0f; },
                                sh.wg, bank);
  token = st >= 0 ? L.id(st) : tok0;
}

__global__ __launch_bounds__(kNT) void k_sample(RowParams P, RowPtrs Q) {
  __shared__ SampleShared sh;
  int bank = 0;
  const int row = blockIdx.x;
  const int t = (int)threadIdx.x;
  const int n = P.n;
  const bool t1 = (P.flags & kFlagTIsOne) != 0;
  const bool vec = (P.flags & kFlagVecSrc) != 0;
  const float* xr = Q.src + (int64_t)row * P.src_stride;

  // ---- 1. row maximum from the partials (sampler.zig:80-81)
  float m = -kInf;
  for (int i = t; i < P.nparts; i += kNT) m = fmaxf(m, Q.maxpart[(int64_t)row * P.nparts + i]);
  m = wg_fmax<kNT>(m, sh.wg, bank);

  // ---- 2. exact sequential normaliser + candidate collection (:83-88)
  if (t == 0) sh.cand_count = 0;
  __syncthreads();
  float s = 0.0f;
  for (int base = 0; base < n; base += kTile) {
    float v[kV], e[kV];
    const int pos = base + t * kV;
    load4(xr, pos, n, vec, v);
#pragma unroll
    for (int k = 0; k < kV; ++k) {
      e[k] = row_exp(v[k], m, P.temperature, t1);
      if (pos + k < n && e[k] >= P.cand_theta) {
        const uint32_t slot = atomicAdd(&sh.cand_count, 1u);
        if (slot < (uint32_t)kCap) sh.cand[slot] = ((uint64_t)__float_as_uint(e[k]) << 32) | (uint32_t)(pos + k);
      }
    }
    int st;
    s = tile_accumulate<kNT, kV, false>(s, e, min(kTile, n - base), -1.0f, st, sh.wg, bank);
  }
  const float S = s;

  uint32_t token = 0, consumed = 0, path = 0;
  float H = 0.0f, total = 0.0f;
  int K = 0;

  // ---- 3. sum <= 0 exit: sampleArgmax of the caller's logits (:89)
  if (S <= 0.0f) {
    token = wg_argmax_row<kNT>(Q.orig + (int64_t)row * P.orig_stride, n, sh.wg, bank);
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

  // ---- 4. candidates -> probabilities -> (p desc, id asc) (:90-100)
  __syncthreads();
  const uint32_t cc = sh.cand_count;
  const bool ovf = cc > (uint32_t)kCap;
  const int c = ovf ? kCap : (int)cc;
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
  __syncthreads();
  lds_bitonic_sort_u64<kNT>(sh.cand, csort);

  // certified prefix: every element outside the list has p <= theta / S
  int M = 0;
  if (!ovf) {
    if (P.cand_theta <= 0.0f) {
      M = c;  // every element was collected
    } else {
      const float p_nc = P.cand_theta / S;
      uint32_t cnt = 0;
      for (int q = t; q < c; q += kNT) cnt += __uint_as_float(~(uint32_t)(sh.cand[q] >> 32)) > p_nc ? 1u : 0u;
      M = (int)wg_sum_sat<kNT>(cnt, 0x7fffffffu, sh.wg, bank);
    }
  }

  const LdsList LL{sh.cand};
  // a complete list bounds everything outside it: e < theta, p <= theta / S
  const float p_nc = ovf ? kInf : P.cand_theta / S;
  K = prefix_filters(LL, M, p_nc, n, P, S, sh, bank);
  const bool typical = P.typical_p > 0.0f && P.typical_p < 1.0f;
  const float u = Q.uniforms[row];
  bool fallback = K < 0;

  if (!fallback) {
    // ---- 5. typical-p on the kept prefix (:128-154)
    for (int q = t; q < kCap; q += kNT) sh.keep[q] = q < K ? 1 : 0;
    __syncthreads();
    if (typical && K == 1) {
      if (t == 0 && LL.p(0) > P.typical_p) sh.keep[0] = 0;
      __syncthreads();
    } else if (typical && K >= 2) {
      path |= kPathEntropy;
      H = entropy_pass(xr, n, m, S, P, sh, bank);
      const int ksort = next_pow2(K);
      for (int q = t; q < ksort; q += kNT) {
        if (q < K) {
          const float p = LL.p(q);
          const float surprise = p > 0.0f ? -log_f32(p) : kInf;
          const float dev = fabsf(surprise - H);
          sh.aux[q] = ((uint64_t)__float_as_uint(dev) << 32) | LL.id(q);
          sh.aux_pos[q] = (uint32_t)q;
        } else {
          sh.aux[q] = ~0ull;
          sh.aux_pos[q] = 0;
        }
      }
      __syncthreads();
      lds_bitonic_sort_kv<kNT>(sh.aux, sh.aux_pos, ksort);
      int st;
      list_accumulate<kNT, 2, false>(0.0f, K, P.typical_p, st,
                                     [&](int d) { return LL.p((int)sh.aux_pos[d]); }, sh.wg, bank);
      if (st >= 0) {
        for (int d = st + t; d < K; d += kNT) sh.keep[sh.aux_pos[d]] = 0;
      }
      __syncthreads();
    }
    // ---- 6. total and draw (:156-168)
    total_and_draw(LL, K, [&](int q) { return sh.keep[q] != 0; }, u, total, token, consumed, sh, bank);

    // ---- outputs
    uint32_t kept = 0;
    for (int q = t; q < K; q += kNT) kept += sh.keep[q];
    kept = wg_sum_sat<kNT>(kept, 0x7fffffffu, sh.wg, bank);
    if (Q.kept_ids || Q.kept_probs) {
      // compact the kept positions in p order (thread-serial over K <= kCap)
      if (t == 0) {
        int o = 0;
        for (int q = 0; q < K && o < P.kept_cap; ++q) {
          if (sh.keep[q]) {
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
  path |= kPathFallback;
  if (!(P.flags & kFlagFallback)) {
    if (t == 0) {
      Q.tokens[row] = 0xffffffffu;
      if (Q.consumed) Q.consumed[row] = 0;
      if (Q.status) Q.status[row] = path | kPathError;
    }
    return;
  }
  const int64_t fo = (int64_t)row * n;
  uint32_t* Ak = Q.fb + 0 * (int64_t)P.rows * n + fo;
  uint32_t* Av = Q.fb + 1 * (int64_t)P.rows * n + fo;
  uint32_t* Bk = Q.fb + 2 * (int64_t)P.rows * n + fo;
  uint32_t* Bv = Q.fb + 3 * (int64_t)P.rows * n + fo;
  uint32_t* Ck = Q.fb + 4 * (int64_t)P.rows * n + fo;
  uint32_t* Cv = Q.fb + 5 * (int64_t)P.rows * n + fo;
  uint8_t* mask = Q.fb_mask + fo;
  for (int base = 0; base < n; base += kTile) {
    float v[kV];
    const int pos = base + t * kV;
    load4(xr, pos, n, vec, v);
#pragma unroll
    for (int k = 0; k < kV; ++k) {
      if (pos + k < n) {
        const float p = row_exp(v[k], m, P.temperature, t1) / S;
        Ak[pos + k] = ~__float_as_uint(p);
        Av[pos + k] = (uint32_t)(pos + k);
      }
    }
  }
  __threadfence();
  __syncthreads();
  wg_radix_sort_pairs<kNT>(Ak, Av, Bk, Bv, n, sh.radix);
  __threadfence();
  __syncthreads();
  const GlobalList GL{Ak, Av};
  K = prefix_filters(GL, n, kInf, n, P, S, sh, bank);  // M = n: never -1
  if (K < 0) K = 0;
  if (typical && K >= 2) {
    path |= kPathEntropy;
    H = entropy_pass(xr, n, m, S, P, sh, bank);
    for (int i = t; i < n; i += kNT) mask[i] = 0;
    __threadfence();
    __syncthreads();
    for (int q = t; q < K; q += kNT) mask[Av[q]] = 1;
    __threadfence();
    __syncthreads();
    // selected ids in index order with their dev keys (stream compaction)
    int written = 0;
    for (int base = 0; base < n; base += kNT) {
      const int i = base + t;
      const bool sel = i < n && mask[i] == 1;
      const uint32_t before = wg_excl_scan_sat<kNT>(sel ? 1u : 0u, 0x7fffffffu, sh.wg, bank);
      if (sel) {
        const float p = row_exp(xr[i], m, P.temperature, t1) / S;
        const float surprise = p > 0.0f ? -log_f32(p) : kInf;
        Bk[written + before] = __float_as_uint(fabsf(surprise - H));
        Bv[written + before] = (uint32_t)i;
      }
      written += (int)wg_sum_sat<kNT>(sel ? 1u : 0u, 0x7fffffffu, sh.wg, bank);
    }
    __threadfence();
    __syncthreads();
    wg_radix_sort_pairs<kNT>(Bk, Bv, Ck, Cv, written, sh.radix);
    __threadfence();
    __syncthreads();
    int st;
    list_accumulate<kNT, 2, false>(
        0.0f, written, P.typical_p, st,
        [&](int d) { return row_exp(xr[Bv[d]], m, P.temperature, t1) / S; }, sh.wg, bank);
    const int keep_n = st >= 0 ? st : written;
    for (int d = t; d < keep_n; d += kNT) mask[Bv[d]] = 2;
    __threadfence();
    __syncthreads();
    total_and_draw(GL, K, [&](int q) { return mask[Av[q]] == 2; }, u, total, token, consumed, sh, bank);
  } else if (typical && K == 1) {
    const bool k0 = !(GL.p(0) > P.typical_p);
    total_and_draw(GL, K, [&](int q) { return k0; }, u, total, token, consumed, sh, bank);
  } else {
    total_and_draw(GL, K, [&](int q) { return true; }, u, total, token, consumed, sh, bank);
  }
  // outputs (kept list compaction is thread-serial: diagnostic use only)
  const bool use_mask = typical && K >= 2;
  uint32_t kept = 0;
  for (int q = t; q < K; q += kNT) {
    bool kq = use_mask ? mask[Av[q]] == 2 : (typical && K == 1 ? !(GL.p(0) > P.typical_p) : true);
    kept += kq ? 1u : 0u;
  }
  kept = wg_sum_sat<kNT>(kept, 0x7fffffffu, sh.wg, bank);
  if (t == 0) {
    if (Q.kept_ids || Q.kept_probs) {
      int o = 0;
      for (int q = 0; q < K && o < P.kept_cap; ++q) {
        bool kq = use_mask ? mask[Av[q]] == 2 : (typical && K == 1 ? !(GL.p(0) > P.typical_p) : true);
        if (kq) {
          if (Q.kept_ids) Q.kept_ids[(int64_t)row * P.kept_cap + o] = GL.id(q);
          if (Q.kept_probs) Q.kept_probs[(int64_t)row * P.kept_cap + o] = GL.p(q);
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
}

// ---------------------------------------------------------------------------
// k_math_probe: the device exp/log on an array (parity tests of the math).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_math_probe(const float* __restrict__ in, float* __restrict__ out_exp,
                                                   float* __restrict__ out_log, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) {
    const float x = in[i];
    if (out_exp) out_exp[i] = exp_f32(x);
    if (out_log) out_log[i] = log_f32(x);
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
hipError_t launch_math_probe(const float* in, float* out_exp, float* out_log, int64_t n, hipStream_t st) {
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(k_math_probe, dim3((unsigned)blocks), dim3(256), 0, st, in, out_exp, out_log, n);
  return hipGetLastError();
}

int max_parts(int n) { return (n + kMaxNT * kMaxPerThread - 1) / (kMaxNT * kMaxPerThread); }

hipError_t launch_penalty(const float* logits, int64_t stride, int rows, int n, const uint32_t* prev,
                          int n_prev, int64_t prev_stride, int window, float penalty, float* out,
                          hipStream_t st) {
  dim3 grid(max_parts(n), rows);
  hipLaunchKernelGGL(k_penalty, grid, dim3(kMaxNT), 0, st, logits, stride, n, prev, n_prev,
                     prev_stride, window, penalty, out);
  return hipGetLastError();
}

hipError_t launch_rowmax(const float* logits, int64_t stride, int rows, int n, bool vec, float* part,
                         hipStream_t st) {
  const int np = max_parts(n);
  dim3 grid(np, rows);
  hipLaunchKernelGGL(k_rowmax, grid, dim3(kMaxNT), 0, st, logits, stride, n, np, vec ? 1 : 0, part);
  return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, int64_t stride, int rows, int n, uint32_t* tokens,
                         uint8_t* consumed, uint32_t* kept_count, hipStream_t st) {
  hipLaunchKernelGGL(k_argmax, dim3(rows), dim3(kNT), 0, st, logits, stride, n, tokens, consumed,
                     kept_count);
  return hipGetLastError();
}

hipError_t launch_sample(const RowParams& P, const RowPtrs& Q, hipStream_t st) {
  hipLaunchKernelGGL(k_sample, dim3(P.rows), dim3(kNT), 0, st, P, Q);
  return hipGetLastError();
}

}  // namespace llz
