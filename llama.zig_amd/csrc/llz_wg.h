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
// global memory.  (k0, v0) is the input and, after the four passes, the
// output; (k1, v1) is the ping-pong buffer.  Equal keys keep input order.
struct RadixScratch {
  uint32_t base[256];
  uint32_t cnt[16][256];  // per-wave digit counts of one tile
};

template <int NT>
__device__ void wg_radix_sort_pairs(uint32_t* k0, uint32_t* v0, uint32_t* k1, uint32_t* v1, int n,
                                    RadixScratch& rs) {
  static_assert(NT % kWave == 0 && NT / kWave <= 16 && NT >= 256, "radix sort layout");
  constexpr int W = NT / kWave;
  const int t = (int)threadIdx.x;
  const int w = wave_id();
  const uint64_t lt_mask = (lane_id() == 0) ? 0ull : (~0ull >> (kWave - lane_id()));
  uint32_t *src_k = k0, *src_v = v0, *dst_k = k1, *dst_v = v1;
  for (int shift = 0; shift < 32; shift += 8) {
    // 1. histogram
    for (int d = t; d < 256; d += NT) rs.base[d] = 0;
    __syncthreads();
    for (int i = t; i < n; i += NT) atomicAdd(&rs.base[(src_k[i] >> shift) & 255u], 1u);
    __syncthreads();
    // 2. exclusive scan of the 256 counts (one wave, 4 per lane)
    if (w == 0) {
      uint32_t c[4], s = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) { c[q] = rs.base[lane_id() * 4 + q]; s += c[q]; }
      uint32_t incl = s;
#pragma unroll
      for (int d = 1; d < kWave; d <<= 1) {
        uint32_t o = __shfl_up(incl, d, kWave);
        if (lane_id() >= d) incl += o;
      }
      uint32_t run = incl - s;
#pragma unroll
      for (int q = 0; q < 4; ++q) { rs.base[lane_id() * 4 + q] = run; run += c[q]; }
    }
    __syncthreads();
    // 3. stable scatter, one element per thread per tile, tiles in order
    for (int tile = 0; tile < n; tile += NT) {
      for (int d = t; d < 256 * W; d += NT) (&rs.cnt[0][0])[d] = 0;
      __syncthreads();
      const int i = tile + t;
      const bool valid = i < n;
      uint32_t key = 0, val = 0, dig = 0;
      if (valid) {
        key = src_k[i];
        val = src_v[i];
        dig = (key >> shift) & 255u;
      }
      // lanes of this wave with the same digit
      uint64_t peers = __ballot(valid);
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const uint64_t bb = __ballot(valid && ((dig >> b) & 1u));
        peers &= ((dig >> b) & 1u) ? bb : ~bb;
      }
      const uint32_t rank_in_wave = (uint32_t)__popcll(peers & lt_mask);
      if (valid && rank_in_wave == 0) rs.cnt[w][dig] = (uint32_t)__popcll(peers);
      __syncthreads();
      if (valid) {
        uint32_t off = rs.base[dig] + rank_in_wave;
        for (int ww = 0; ww < w; ++ww) off += rs.cnt[ww][dig];
        dst_k[off] = key;
        dst_v[off] = val;
      }
      __syncthreads();
      for (int d = t; d < 256; d += NT) {
        uint32_t s = 0;
        for (int ww = 0; ww < W; ++ww) s += rs.cnt[ww][d];
        rs.base[d] += s;
      }
      __syncthreads();
    }
    uint32_t* tk = src_k; src_k = dst_k; dst_k = tk;
    uint32_t* tv = src_v; src_v = dst_v; dst_v = tv;
    // make this pass's global writes visible to the next pass's reads
    __threadfence_block();
    __syncthreads();
  }
}

}  // namespace llz
