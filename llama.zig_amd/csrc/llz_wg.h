// llz_wg.h -- workgroup primitives for one-row-per-workgroup kernels on
// CDNA (64-lane wavefronts): saturating reductions and scans, broadcasts,
// an LDS bitonic sort of 64-bit keys, and a stable LSD radix sort of
// (u32 key, u32 value) pairs in global memory.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llz {

constexpr int kWave = 64;

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }
__device__ __forceinline__ int wave_id() { return (int)(threadIdx.x / kWave); }

// Workgroup barrier that orders LDS only: outstanding global loads (for
// example prefetches) stay in flight.  Code that hands data between threads
// through global memory uses __syncthreads() (or __threadfence()) instead.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Saturating u32 add: results stay <= cap.
__device__ __forceinline__ uint32_t sat_add(uint32_t a, uint32_t b, uint32_t cap) {
  uint32_t s = a + b;  // a, b <= cap <= 2^30, no wrap
  return s < cap ? s : cap;
}

// DPP cross-lane moves (register speed, no LDS round trip).  CTRL values:
// row_shr:n = 0x110+n, wave_shr:1 = 0x138, row_bcast:15 = 0x142,
// row_bcast:31 = 0x143.  Lanes that are masked off, or that read outside
// their row with bound_ctrl set, receive `old`.
template <int CTRL, int ROW_MASK, int BANK_MASK, bool BC>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t old, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROW_MASK, BANK_MASK, BC);
}

// Wave64 inclusive scan for an associative op with identity `id` (the
// row_shr 1/2/3, row_shr 4 and 8, row_bcast 15 and 31 sequence).
template <typename Op>
__device__ __forceinline__ uint32_t wave_incl_scan_op(uint32_t x, uint32_t id, Op op) {
  uint32_t s = x;
  s = op(s, dpp_u32<0x111, 0xf, 0xf, true>(id, x));
  s = op(s, dpp_u32<0x112, 0xf, 0xf, true>(id, x));
  s = op(s, dpp_u32<0x113, 0xf, 0xf, true>(id, x));
  s = op(s, dpp_u32<0x114, 0xf, 0xe, false>(id, s));
  s = op(s, dpp_u32<0x118, 0xf, 0xc, false>(id, s));
  s = op(s, dpp_u32<0x142, 0xa, 0xf, false>(id, s));
  s = op(s, dpp_u32<0x143, 0xc, 0xf, false>(id, s));
  return s;
}

// A wave's ballot of a bool.  HIP's __ballot takes an int, and the compiler
// then rebuilds the mask of a compound condition through a vector register.
__device__ __forceinline__ uint64_t bal64(bool b) { return __builtin_amdgcn_ballot_w64(b); }

__device__ __forceinline__ uint32_t lane_readlast(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, kWave - 1);
}

// Inclusive prefix (saturating) within a wave.
__device__ __forceinline__ uint32_t wave_incl_scan_sat(uint32_t v, uint32_t cap) {
  return wave_incl_scan_op(v, 0u, [cap](uint32_t a, uint32_t b) { return sat_add(a, b, cap); });
}

// The previous lane's value (lane 0 gets 0).
__device__ __forceinline__ uint32_t wave_shift_up1(uint32_t v) { return dpp_u32<0x138, 0xf, 0xf, true>(0u, v); }

__device__ __forceinline__ uint32_t wave_sum_sat(uint32_t v, uint32_t cap) {
  return lane_readlast(wave_incl_scan_sat(v, cap));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  return lane_readlast(wave_incl_scan_op(v, 0u, [](uint32_t a, uint32_t b) { return a > b ? a : b; }));
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  return lane_readlast(
      wave_incl_scan_op(v, 0xffffffffu, [](uint32_t a, uint32_t b) { return a < b ? a : b; }));
}

// Shared scratch for the workgroup reductions.  Two banks alternate so a
// reduction needs one barrier (the next reduction writes the other bank).
template <int NT>
struct WgScratch {
  static constexpr int W = NT / kWave;
  uint32_t red[2][W];
  float fb[2][4];
  uint32_t ub[2][4];
  float sw[W];  // per-wave float results (tile_accumulate_fn's events)
  int bank;
};

template <int NT>
__device__ __forceinline__ uint32_t wg_sum_sat(uint32_t v, uint32_t cap, WgScratch<NT>& sh, int& bank) {
  v = wave_sum_sat(v, cap);
  if (lane_id() == 0) sh.red[bank][wave_id()] = v;
  lds_barrier();
  uint32_t t = 0;
#pragma unroll
  for (int w = 0; w < WgScratch<NT>::W; ++w) t = sat_add(t, sh.red[bank][w], cap);
  bank ^= 1;
  return t;
}

template <int NT>
__device__ __forceinline__ uint32_t wg_max_u32(uint32_t v, WgScratch<NT>& sh, int& bank) {
  v = wave_max_u32(v);
  if (lane_id() == 0) sh.red[bank][wave_id()] = v;
  lds_barrier();
  uint32_t t = 0;
#pragma unroll
  for (int w = 0; w < WgScratch<NT>::W; ++w) t = max(t, sh.red[bank][w]);
  bank ^= 1;
  return t;
}

template <int NT>
__device__ __forceinline__ uint32_t wg_min_u32(uint32_t v, WgScratch<NT>& sh, int& bank) {
  v = wave_min_u32(v);
  if (lane_id() == 0) sh.red[bank][wave_id()] = v;
  lds_barrier();
  uint32_t t = 0xffffffffu;
#pragma unroll
  for (int w = 0; w < WgScratch<NT>::W; ++w) t = min(t, sh.red[bank][w]);
  bank ^= 1;
  return t;
}

// Exclusive prefix (saturating) of one value per thread, in thread order.
template <int NT>
__device__ __forceinline__ uint32_t wg_excl_scan_sat(uint32_t v, uint32_t cap, WgScratch<NT>& sh, int& bank) {
  const uint32_t incl = wave_incl_scan_sat(v, cap);
  if (lane_id() == kWave - 1) sh.red[bank][wave_id()] = incl;
  // exclusive = the previous lane's inclusive value: exact whenever it is
  // below the cap (a saturated prefix only ever reads as "at least cap")
  const uint32_t excl_in_wave = wave_shift_up1(incl);
  lds_barrier();
  uint32_t before = 0;
  const int w = wave_id();
  for (int i = 0; i < w; ++i) before = sat_add(before, sh.red[bank][i], cap);
  bank ^= 1;
  return sat_add(before, excl_in_wave, cap);
}

// Broadcast a float and a u32 written by one thread.
template <int NT>
__device__ __forceinline__ void wg_bcast(bool writer, float& f, uint32_t& u, WgScratch<NT>& sh, int& bank) {
  if (writer) {
    sh.fb[bank][0] = f;
    sh.ub[bank][0] = u;
  }
  lds_barrier();
  f = sh.fb[bank][0];
  u = sh.ub[bank][0];
  bank ^= 1;
}

// Bitonic sort, ascending, of `n` (power of two) u64 keys in LDS.
template <int NT>
__device__ void lds_bitonic_sort_u64(uint64_t* a, int n) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = (int)threadIdx.x; i < n; i += NT) {
        const int p = i ^ j;
        if (p > i) {
          const uint64_t x = a[i], y = a[p];
          const bool up = (i & k) == 0;
          if ((x > y) == up) {
            a[i] = y;
            a[p] = x;
          }
        }
      }
      lds_barrier();
    }
  }
}

// Stable LSD radix sort (8-bit digits, ascending keys) of n pairs held in
// global memory, by one workgroup.  (k0, v0) is the input and the output;
// (k1, v1) is the ping-pong buffer.  Equal keys keep input order.
//
// The digits are those of key - kbase (kbase: at most the smallest key, so
// that the order is the keys' own): keys that span few values then share
// their high digits.  One read of the keys counts the digits of all four
// passes; a pass whose digit is the same for every key moves nothing and is
// skipped (it would keep the order).  A pass handles tiles of kRadixRounds * NT elements:
// round r of a tile holds elements tile + r NT + t, so (round, wave, lane)
// order is input order.  Each round ranks its elements within their wave
// (lanes with the same digit found by eight ballots), the counts of every
// (round, wave) go to LDS, and one scan per digit turns them into the
// elements' places in the tile ordered by digit.  The tile is staged in LDS
// in that order and written out in it: each digit's elements of the tile go
// to consecutive global addresses, so the writes are runs, not scattered
// words.
constexpr int kRadixRounds = 8;

struct RadixScratch {
  uint32_t hist[4][256];                  // digit counts of the whole input, per pass
  uint32_t base[256];                     // next output offset per digit
  int32_t delta[256];                     // tile: output offset minus tile place, per digit
  uint32_t wsum[4];                       // tile: digit-total scan, per wave of the scan
  uint16_t cnt[kRadixRounds][8][256];     // per (round, wave): digit counts, then tile places (< 2^16)
  uint32_t stage_k[kRadixRounds * 512];   // the tile ordered by digit
  uint32_t stage_v[kRadixRounds * 512];
};

template <int NT>
__device__ void wg_radix_sort_pairs(uint32_t* k0, uint32_t* v0, uint32_t* k1, uint32_t* v1, int n,
                                    RadixScratch& rs, uint32_t kbase = 0u) {
  static_assert(NT % kWave == 0 && NT / kWave <= 8 && NT >= 256 && NT <= 512, "radix sort layout");
  static_assert(kRadixRounds * 512 <= 65536, "tile places fit 16 bits");
  constexpr int W = NT / kWave;
  constexpr int R = kRadixRounds;
  constexpr int TILE = R * NT;
  const int t = (int)threadIdx.x;
  const int w = wave_id();
  const int lane = lane_id();
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
  if (n <= 1) return;

  // digit counts of all four passes
  for (int d = t; d < 4 * 256; d += NT) (&rs.hist[0][0])[d] = 0;
  __syncthreads();
  for (int i = t; i < n; i += NT) {
    const uint32_t key = k0[i] - kbase;
    atomicAdd(&rs.hist[0][key & 255u], 1u);
    atomicAdd(&rs.hist[1][(key >> 8) & 255u], 1u);
    atomicAdd(&rs.hist[2][(key >> 16) & 255u], 1u);
    atomicAdd(&rs.hist[3][key >> 24], 1u);
  }
  __syncthreads();

  uint32_t *src_k = k0, *src_v = v0, *dst_k = k1, *dst_v = v1;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 8 * pass;
    // a digit shared by every key: nothing moves
    bool constant = false;
    for (int d = 0; d < 256; ++d) constant = constant || rs.hist[pass][d] == (uint32_t)n;
    if (constant) continue;
    // exclusive scan of the pass's counts (one wave, four digits per lane)
    if (w == 0) {
      uint32_t c[4], sum = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) { c[q] = rs.hist[pass][lane * 4 + q]; sum += c[q]; }
      uint32_t incl = sum;
#pragma unroll
      for (int d = 1; d < kWave; d <<= 1) {
        const uint32_t o = __shfl_up(incl, d, kWave);
        if (lane >= d) incl += o;
      }
      uint32_t run = incl - sum;
#pragma unroll
      for (int q = 0; q < 4; ++q) { rs.base[lane * 4 + q] = run; run += c[q]; }
    }
    // the tile's elements, loaded one tile ahead (the barriers inside the
    // loop order LDS only, so these loads and the previous tile's writes
    // stay in flight across them)
    uint32_t nk[R], nv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = r * NT + t;
      nk[r] = i < n ? src_k[i] : 0u;
      nv[r] = i < n ? src_v[i] : 0u;
    }
    for (int tile = 0; tile < n; tile += TILE) {
      const int tn = min(TILE, n - tile);
      uint32_t key[R], val[R], dig[R], rank[R];
      bool valid[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        valid[r] = tile + r * NT + t < n;
        key[r] = nk[r];
        val[r] = nv[r];
      }
      if (tile + TILE < n) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int i = tile + TILE + r * NT + t;
          nk[r] = i < n ? src_k[i] : 0u;
          nv[r] = i < n ? src_v[i] : 0u;
        }
      }
      // zero the tile's counts (the previous tile's last reads are done)
      uint4* cz = reinterpret_cast<uint4*>(&rs.cnt[0][0][0]);
      for (int d = t; d < R * 8 * 256 / 8; d += NT) cz[d] = make_uint4(0u, 0u, 0u, 0u);
      lds_barrier();
#pragma unroll
      for (int r = 0; r < R; ++r) {
        dig[r] = ((key[r] - kbase) >> shift) & 255u;
        // lanes of this wave with the same digit
        uint64_t peers = bal64(valid[r]);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          const uint64_t bb = bal64(((dig[r] >> b) & 1u) != 0u);
          peers &= ((dig[r] >> b) & 1u) ? bb : ~bb;
        }
        rank[r] = (uint32_t)__popcll(peers & lt_mask);
        if (valid[r] && rank[r] == 0) rs.cnt[r][w][dig[r]] = (uint16_t)__popcll(peers);
      }
      lds_barrier();
      // per digit (thread d < 256, waves 0 .. 3): its tile total, the tile
      // place where its elements start (a scan over digits), then each
      // (round, wave)'s place
      uint32_t tot = 0, incl = 0;
      if (t < 256) {
#pragma unroll 8
        for (int rw = 0; rw < R * W; ++rw) tot += rs.cnt[rw / W][rw % W][t];
        incl = wave_incl_scan_op(tot, 0u, [](uint32_t a, uint32_t b) { return a + b; });
        if (lane == kWave - 1) rs.wsum[w] = incl;
      }
      lds_barrier();
      if (t < 256) {
        const int d = t;
        uint32_t start = incl - tot;
        for (int ww = 0; ww < w; ++ww) start += rs.wsum[ww];
        uint32_t run = start;
#pragma unroll 8
        for (int rw = 0; rw < R * W; ++rw) {
          uint16_t* c = &rs.cnt[rw / W][rw % W][d];
          const uint32_t v = *c;
          *c = (uint16_t)run;
          run += v;
        }
        rs.delta[d] = (int32_t)rs.base[d] - (int32_t)start;
        rs.base[d] += tot;
      }
      lds_barrier();
      // stage the tile in digit order
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (valid[r]) {
          const uint32_t place = rs.cnt[r][w][dig[r]] + rank[r];
          rs.stage_k[place] = key[r];
          rs.stage_v[place] = val[r];
        }
      }
      lds_barrier();
      // write it out in that order: runs of consecutive addresses per digit
      for (int i = t; i < tn; i += NT) {
        const uint32_t k = rs.stage_k[i];
        const int32_t off = rs.delta[((k - kbase) >> shift) & 255u] + i;
        dst_k[off] = k;
        dst_v[off] = rs.stage_v[i];
      }
      lds_barrier();
    }
    uint32_t* tk = src_k; src_k = dst_k; dst_k = tk;
    uint32_t* tv = src_v; src_v = dst_v; dst_v = tv;
    // make this pass's global writes visible to the next pass's reads
    __threadfence_block();
    __syncthreads();
  }
  // an odd number of passes left the result in (k1, v1): copy it back
  if (src_k != k0) {
    for (int i = t; i < n; i += NT) {
      k0[i] = src_k[i];
      v0[i] = src_v[i];
    }
    __threadfence_block();
    __syncthreads();
  }
}

}  // namespace llz
