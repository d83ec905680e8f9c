// llz_fast.h -- single-pass row statistics: the row maximum, the exact
// sequential f32 normaliser and the candidate list (sampler.zig:80-88) with
// one HBM read per logit.
//
// One 512-thread workgroup owns a row.  Wave w owns the 256-element segments
// w, w + W, w + 2W, ... (interleaved, so the costly start of the row is
// shared by every wave); its first KV segments stay in VGPRs (one float4 per
// lane per segment), the next KL in LDS.
//
// Phase L (as the loads land, a window of kLoadWindow in flight per wave):
// per-lane running maximum; the estimate
//     q = exp2(v * RN(log2(e)/T) - c_w),   c_w = RN(m_w * RN(log2(e)/T))
// with m_w the maximum of the wave's first segment, stored over v; the
// segment sum of q.
// Phase M: the row maximum m; R_w = exp2(c_w - m * RN(log2(e)/T)) turns q into
// q * R_w ~ e = exp((v - m) / T).  A prefix of the segment sums predicts the
// binade of the running sum at every segment; a segment whose predicted
// range [P(1 - d), P_end(1 + d)] stays inside one binade j is PLAIN, any
// other is EXACT.
// Phase S: PLAIN segments round every term on the binade's grid
// u = 2^(j-23): with sc = R_w 2^(23-j), fma(q, sc(1 -+ eps), 1.5*2^23) gives
// RN(q sc (1 -+ eps)) as an integer.  When both agree the true RN(e / u) is
// that integer and is not a tie; the others (and the large terms and the
// candidates) are "special": queued, re-read, evaluated with the exact exp
// (llz_math.h) and corrected.  A segment holding a tie becomes PLAIN_TIE: its
// ties add units that depend only on the parity of the integer it starts at.
// Phase F+X: EXACT segments are re-read and evaluated exactly into LDS, with
// per-lane prefix tables of their roundings on the grids they span.
// Phase B: the walk's entries (runs of PLAIN segments on one grid, PLAIN_TIE
// and EXACT segments).
// Phase C: one wave walks the entries in index order: runs add their integer
// sums while the running sum stays in their binade; an EXACT segment is
// resolved from its tables, replaying in floating point only the lane that
// holds an event (a tie or a binade crossing); anything the tables do not
// cover takes the exact parallel accumulation (wave_accumulate, llz_norm.h).
//
// Error bound of the estimate relative to the reference's term e =
// exp(RN(RN(v - m) / T)) for the terms that can round to a non-zero integer
// (X = (v - m) log2(e) / T, |X| <= 25 - j): the reference's own two
// roundings of its argument (one when T == 1: RN(x / 1) is exact) and the
// rounding of log2(e)/T contribute 3|X| 2^-24 (2|X| when T == 1, in log2
// units); with B_w = c_w - m RN(log2(e)/T) (|B_w| <= 64, checked; the kernel
// bounds with the wave's rounded value |aw| = |RN(B_w)|), the rounding of
// v RN(log2(e)/T) - c_w adds at most (|X| + |B_w|) 2^-24 and that of the
// argument of R_w at most |B_w| 2^-24, so together ln2 (4|X| + 2|B_w|) 2^-24
// (3|X| when T == 1), taken with 3 units to spare; the two hardware exp2
// (<= 2^-23 each), the final multiply (2^-24) and the reference exp
// (< 2^-23) add < 2^-21.  eps(j) is twice that bound.  For |X| > 25 - j the
// terms are below 1/4 of the grid and round to 0 on both sides.
//
// Anything the fast path cannot certify (an unpredicted binade crossing, a
// grid mismatch, a queue overflow, a row longer than the resident capacity)
// sets `fail`; the caller then runs the streaming normaliser instead.
#pragma once

#include "llz_accum.h"
#include "llz_exact.h"
#include "llz_internal.h"
#include "llz_math.h"
#include "llz_norm.h"
#include "llz_wg.h"

namespace llz {
namespace fastp {
constexpr int NT = 512;
constexpr int W = NT / kWave;       // 8 waves
constexpr int SEG = 256;            // elements per segment: one float4 per lane
constexpr int KV = 45;              // register-resident segments per wave
constexpr int KL = 18;              // LDS-resident segments per wave
constexpr int SPWMAX = KV + KL;     // segments per wave at most (<= 64: one lane each)
constexpr int GMAX = W * SPWMAX;    // 504 segments = 129024 logits
constexpr int QCAP = 128;           // special queue capacity per wave (flushed when full)
constexpr int kLoadWindow = 6;     // phase L: segment loads in flight per wave
constexpr int DCAP = 48;            // EXACT segments evaluated per round
constexpr int NG = 6;               // grids tabulated per EXACT segment at most
// Relative margin of the binade prediction.  The walk checks every
// prediction (a wrong one sends the row to the streaming normaliser, exact
// but several times slower, and one such row costs the whole launch), so
// the margin trades EXACT segments against such rows.  What separates the
// reference's sequential f32 sum from the estimate's sum is mostly the
// terms below half a grid unit, which the reference drops: on the headline
// data a margin of 2^-13 left rows uncertified, 2^-12 none; 2^-11 keeps
// twice that.
constexpr float DELTA = 0x1p-11f;
constexpr float MAGIC = 12582912.0f;            // 1.5 * 2^23
constexpr uint32_t MAGIC_BITS = 0x4b400000u;    // its bit pattern
// PLAIN: integer sum on one grid; PLAIN_TIE: the same, plus the units its
// ties add (sbump);
// EXACT_PRED: predicted binade change, its candidates not collected yet;
// EXACT_DONE: the same, collected.
enum : uint8_t { PLAIN = 0, EXACT_PRED = 1, PLAIN_TIE = 2, EXACT_DONE = 3 };
static_assert(SPWMAX <= 64, "segment metadata is held one segment per lane");
static_assert(DCAP <= 127, "slots are stored as int8");
static_assert(GMAX <= 8 * 64, "the combine holds eight segments per lane");
}  // namespace fastp

// EXACT segments: exact terms, per-lane inclusive prefixes of their
// roundings on grids sj .. sj + sng - 1, and the lanes holding a tie.
// and the walk's entries in index order: a run of PLAIN segments on one
// binade, a PLAIN_TIE segment, or an EXACT segment.  Word a: type (bits
// 0-1), segment (2-11), binade + 128 (16-23), tie units (24-31); word b: the
// integer sum of a run or a PLAIN_TIE segment.
struct ExactSlots {
  float dump[fastp::DCAP][fastp::SEG];
  uint32_t pref[fastp::DCAP][fastp::NG][kWave];
  uint64_t tmask[fastp::DCAP][fastp::NG];
  uint32_t ent_a[fastp::GMAX];
  uint32_t ent_b[fastp::GMAX];
};

struct FastShared {
  union {
    float data[fastp::W][fastp::KL][fastp::SEG];  // LDS-resident segments (q), phases L and S
    ExactSlots x;                                 // after phase S
    struct {
      ExactSlots x;
      float4 ctab[fastp::W][kWave];               // phase S: the register batches' per-segment constants,
    } s;                                          //   past everything phases F+X .. C write
  } u;
  union {
    float aseg[fastp::GMAX];                    // segment sums of q (phases L, M)
    alignas(16) uint32_t ssum4[fastp::W * 64][4];  // PLAIN: integer sum on grid sj in four parts, plus
                                                //   4 * 64 * MAGIC_BITS (mod 2^32) (from phase S; room
                                                //   for every wave's 64th segment: stored unguarded)
  } v;
  int8_t sj[fastp::GMAX];                       // PLAIN: its binade; EXACT: first binade tabulated
  uint8_t sng[fastp::GMAX];                     // EXACT: number of binades tabulated
  uint8_t sflag[fastp::GMAX];
  int8_t sdump[fastp::GMAX];                    // EXACT: slot in `dump`, or -1
  uint8_t sbump[fastp::GMAX];                   // PLAIN_TIE: units its ties add when the segment
                                                //   starts at an even (bits 0-3) or odd (4-7) integer
  uint32_t qpos[fastp::W][fastp::QCAP];         // special queue: position (bits 0-30) and the parity of its
                                                //   segment's integer sum before it (bit 31, lower brackets)
  int16_t slotseg[fastp::DCAP];                 // segment held by each EXACT slot
  float mw[fastp::W];
  float cw[fastp::W];
  float bw[fastp::W];       // per wave: |aw|, the R_w argument's magnitude (error bound)
  uint32_t nanw[fastp::W];
  float wtot[fastp::W];     // per wave: sum of its scaled segment sums
  uint32_t wflag[fastp::W]; //   bit 0: not certifiable, bit 1: candidate flood
  int wnex[fastp::W];       //   number of its EXACT segments
  uint32_t ncand;
  int nslot;      // EXACT slots in use this round
  uint32_t fail;
  uint32_t flood;
  int next_e;     // combine: first entry not consumed yet
  int ne;         // combine: number of entries
  float s_run;    // combine: running sum at next_g
  int done;
  uint32_t diag;  // kPathWalkRounds / kPathResolveGeneric (diagnostics for the row's status)
  float qsum[fastp::W];  // token-only rows: per wave, the sum of its estimates q
  float tx[fastp::W];    // token-only typical-p rows: per wave, sum of q (log2 q + aw)
  float txa[fastp::W];   //   and of its terms' magnitudes
  float theta2;          // token-only rows: the threshold of a list collected again
  float qwsum[fastp::W];  // token-only rows: per wave, its segments' sums of q times n - their first position
  uint32_t tcand; // token-only rows: candidates collected
  uint32_t tfail; // token-only rows: not certified (the exact phases follow)
};

typedef int llz_i4v __attribute__((ext_vector_type(4)));

// Raw buffer load of 16 bytes (buffer_load_dwordx4 ... offen): address =
// resource base + voffset (VGPR) + soffset (SGPR); reads past the
// resource's byte count return 0.  aux 2 = non-temporal.
__device__ llz_i4v llz_raw_buffer_load_v4i32(llz_i4v rsrc, int voffset, int soffset,
                                             int aux) __asm("llvm.amdgcn.raw.buffer.load.v4i32");

// Buffer resource over `bytes` bytes at `base` (wave-uniform): raw buffer,
// stride 0, gfx9 word 3 (32-bit data format).
__device__ __forceinline__ llz_i4v row_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  llz_i4v r;
  r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r.y = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));
  r.z = __builtin_amdgcn_readfirstlane((int)bytes);
  r.w = 0x00020000;
  return r;
}

// 16 bytes per lane from global memory straight to LDS (lane i writes
// lds_base + 16 i).  Written as inline asm on purpose: the compiler's wait
// insertion does not see it, so it keeps counting only its own loads (issue
// these before them: an older load only makes the compiler's waits
// stronger).  The caller waits with s_waitcnt vmcnt(0) before reading LDS.
__device__ __forceinline__ void dma16(const float* gaddr, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gaddr), "s"(lds_base) : "m0", "memory");
}

// The same from a buffer resource (address as in buf_ld4): reads past the
// resource's byte count write zeros.  Non-temporal.
__device__ __forceinline__ void dma_buf16(llz_i4v rsrc, int voffset, int soffset, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, %3 offen nt lds" ::"v"(voffset), "s"(rsrc), "s"(lds_base),
               "s"(soffset)
               : "m0", "memory");
}

// v_writelane: old with lane `lane` (uniform) replaced by src (uniform).
__device__ int llz_writelane_i32(int src, int lane, int old) __asm("llvm.amdgcn.writelane.i32");

// max(a, b, c) of the values as they are: in IEEE mode a quiet NaN operand
// is skipped, a signalling one makes the result NaN (the compiler's fmaxf
// quiets every operand first, one more instruction each).
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Wait until at most N vector memory loads of this wave are in flight.
template <int N>
__device__ __forceinline__ void lds_dma_wait() {
  static_assert(N >= 0 && N <= 63, "vmcnt holds 0 .. 63");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ float4 buf_ld4(llz_i4v rsrc, int voffset, int soffset) {
  const llz_i4v v = llz_raw_buffer_load_v4i32(rsrc, voffset, soffset, 2);
  return make_float4(__int_as_float(v.x), __int_as_float(v.y), __int_as_float(v.z), __int_as_float(v.w));
}

__device__ __forceinline__ float4 ld_nt4(const float* p) {
  const llz_f4v v = __builtin_nontemporal_load(reinterpret_cast<const llz_f4v*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}

// Segment load: a full, 16-byte aligned segment as one float4 per lane;
// otherwise per element, absent positions (>= n) as -inf.
__device__ __forceinline__ float4 ld_seg(const float* xr, int pos, int n, bool vec) {
  if (vec && pos + 4 <= n) return ld_nt4(xr + pos);
  float4 v;
  v.x = pos + 0 < n ? xr[pos + 0] : -__builtin_inff();
  v.y = pos + 1 < n ? xr[pos + 1] : -__builtin_inff();
  v.z = pos + 2 < n ? xr[pos + 2] : -__builtin_inff();
  v.w = pos + 3 < n ? xr[pos + 3] : -__builtin_inff();
  return v;
}

__device__ __forceinline__ float wave_sum_f32(float v) {
  const uint32_t r = wave_incl_scan_op(__float_as_uint(v), 0u, [](uint32_t a, uint32_t b) {
    return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
  });
  return __uint_as_float(lane_readlast(r));
}

// A wave's total of v in lane 63 only, in six folded DPP additions (row
// sums, then rows 0-1 and 2-3, then all four; the other lanes end with
// partial sums).  The order of the additions differs from a lane-order
// scan: for estimates only.
template <int CTRL>
__device__ __forceinline__ float dpp_add_f32(float s) {
  // -0 is the exact identity of f32 addition, so the addition folds into one
  // DPP instruction
  return s + __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-0.0f), __float_as_int(s), CTRL, 0xf, 0xf, true));
}
__device__ __forceinline__ float wave_fold_f32(float v) {
  float s = v;
  s = dpp_add_f32<0x111>(s);  // row_shr:1
  s = dpp_add_f32<0x112>(s);  // row_shr:2
  s = dpp_add_f32<0x114>(s);  // row_shr:4
  s = dpp_add_f32<0x118>(s);  // row_shr:8: lane 15 of each row holds its row's sum
  s = dpp_add_f32<0x142>(s);  // row_bcast:15: lane 63 holds rows 2 + 3
  s = dpp_add_f32<0x143>(s);  // row_bcast:31: lane 63 holds all four rows
  return s;
}


template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xf, 0xf, true);
}

// Sums of four per-lane values over each 16-lane row, transposed: lane
// 16 r + 12 + c ends with the sum of a_c over row r (wrapping u32 adds).
// Eleven instructions, where four wave totals take 24.
__device__ __forceinline__ uint32_t row_sums4(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3) {
  const int lane = lane_id();
  const bool odd = (lane & 1) != 0, b1 = (lane & 2) != 0;
  // lane pairs (quad_perm 1,0,3,2): the even lane ends with the pair's sum of
  // a0 (a2), the odd lane with that of a1 (a3)
  const uint32_t s01 = (odd ? a1 : a0) + dpp_u32<0xB1>(odd ? a0 : a1);
  const uint32_t s23 = (odd ? a3 : a2) + dpp_u32<0xB1>(odd ? a2 : a3);
  // quads (quad_perm 2,3,0,1): lane 4 i + c ends with the quad's sum of a_c
  uint32_t t = (b1 ? s23 : s01) + dpp_u32<0x4E>(b1 ? s01 : s23);
  // the row's four quads (row_shr 4, then 8)
  t = t + dpp_u32<0x114>(t);
  t = t + dpp_u32<0x118>(t);
  return t;
}

__device__ __forceinline__ float wave_max_f32(float v) {
  const uint32_t r = wave_incl_scan_op(__float_as_uint(v), __float_as_uint(-__builtin_inff()),
                                       [](uint32_t a, uint32_t b) {
                                         return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
                                       });
  return __uint_as_float(lane_readlast(r));
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
  return lane_readlast(wave_incl_scan_op(v, 0u, [](uint32_t a, uint32_t b) { return a + b; }));
}

// Relative error bound of the estimate for terms that matter on grid j
// (see the header comment), doubled.  bw = |B_w|, the magnitude of the wave's
// rounded R_w argument fma(m, -RN(log2(e)/T), c_w) (at most 64); t1: T == 1,
// where the reference's argument takes one rounding instead of two; xe: the
// estimates' extra error on soft-capped rows (RowParams.est_xe, 0 on others).
__device__ __forceinline__ float fast_eps(int j, float bw, bool t1, float xe) {
  const float ax = (float)(25 - j);
  const float coef = (t1 ? 3.0f : 4.0f) * ax + 2.0f * bw + 3.0f;
  return 2.0f * (0.6931472f * coef * 0x1p-24f + 0x1p-21f + xe);
}

// A float with its mantissa LSB forced to 1 (see the no-tie argument: an
// odd scale never makes q * scale an exact half-integer below 2^15).
__device__ __forceinline__ float odd_mantissa(float x) { return __uint_as_float(__float_as_uint(x) | 1u); }

// Per-grid constants of phase S.
struct GridConst {
  int j;
  float sc_lo, sc_hi;  // R 2^(23-j) (1 -+ eps), odd mantissas
  float tspec;         // rh >= tspec: large term or candidate
};

__device__ __forceinline__ GridConst grid_const(int j, float R, float theta, float bw, bool t1, float xe) {
  GridConst c;
  c.j = j;
  const float sc = ldexpf(R, 23 - j);
  const float eps = fast_eps(j, bw, t1, xe);
  c.sc_lo = odd_mantissa(sc * (1.0f - eps));
  c.sc_hi = odd_mantissa(sc * (1.0f + eps));
  // candidates: e >= theta  =>  e / u >= theta 2^(23-j)
  const float yc = fminf(floorf(ldexpf(theta, 23 - j)), 32768.0f);
  c.tspec = fastp::MAGIC + fmaxf(yc - 1.0f, 0.0f);
  return c;
}

}  // namespace llz
