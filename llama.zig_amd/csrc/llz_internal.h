// llz_internal.h -- types shared by the kernels and the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llz {

typedef float llz_f4v __attribute__((ext_vector_type(4)));  // four floats as one 16-byte access

constexpr int kCandCap = 2048;  // candidate list capacity per row (power of two)
constexpr int kPenMax = 64;     // fused repetition penalty: window entries at most (one per lane)
constexpr int kQovfWave = 4096;  // k_stats special-queue overflow entries per wave
constexpr int kQovfRow = 8 * kQovfWave;  // ... per workgroup (eight waves)
// k_stats workgroups per launch at most (the grid: one per CU, rows beyond
// claimed); the special-queue overflow area has one kQovfRow block per
// workgroup, which samples one row at a time
constexpr int kMaxGrid = 256;
// Full-row fallback buffer sets per call at most (rows beyond wait for one):
// the number of CUs, since k_stats's LDS holds one row-workgroup per CU, so
// no more rows than this can be inside the fallback at once.
constexpr int kFbSlots = 256;
// Split rows (token-only calls of few rows): a row's logits are read by up to
// kSplitMax workgroups at once, each taking one chunk of 2048 nv consecutive
// logits (nv float4 per thread, nv <= kSplitNV) and handing at most kSplitK
// of them to the workgroup that finishes the row.
constexpr int kSplitMax = 64;
constexpr int kSplitK = 64;
constexpr int kSplitNV = 8;
constexpr int kSplitRows = 64;

// RowParams.flags
constexpr uint32_t kFlagTIsOne = 1u;    // temperature == 1.0f exactly: (v - m) / T == v - m
constexpr uint32_t kFlagVecSrc = 2u;    // 16-byte loads are legal on the rows the chain reads
constexpr uint32_t kFlagFallback = 4u;  // the full-row fallback buffers are present
constexpr uint32_t kFlagTokenOnly = 8u;  // no probabilities or row statistics requested: the token alone
constexpr uint32_t kFlagXfExact = 16u;   // transformed rows the single pass cannot estimate: the exact streaming path

// RowParams.xf_src / xf_orig: transforms applied as a row is read
constexpr uint32_t kXfCap = 1u;    // v = tanh(v / cap) * cap   (main.zig:653-658)
constexpr uint32_t kXfScale = 2u;  // v *= inv_scale            (main.zig:663-666)
constexpr uint32_t kXfPen = 4u;    // repetition penalty        (sampler.zig:54-75)

// k_stats's transform modes (a template parameter: each mode its own
// kernel, so the plain rows carry no transform code)
constexpr int kXmNone = 0;   // rows read as they are
constexpr int kXmLight = 1;  // logit scale and/or the fused penalty, applied exactly as each segment lands
constexpr int kXmCap = 2;    // soft-capping: phase L estimates from a closed form, exact values where needed

// per-row status bits (diagnostics)
constexpr uint32_t kPathSumLe0 = 1u;
constexpr uint32_t kPathEntropy = 2u;
constexpr uint32_t kPathFallback = 4u;      // full-row radix sort
constexpr uint32_t kPathNormFallback = 8u;  // streaming normaliser (row not certified by the fast path)
constexpr uint32_t kPathWalkRounds = 16u;    // diagnostic: the walk took more than one round of EXACT slots
constexpr uint32_t kPathResolveGeneric = 32u;  // diagnostic: an event beyond a segment's tabulated grids
constexpr uint32_t kPathTokenOnly = 128u;     // the token certified without the exact normaliser
constexpr uint32_t kPathBuckets = 64u;        // full row without a sort: kept prefix, total and draw by p-key buckets
constexpr uint32_t kPathRecollect = 1u << 16;  // a flooded candidate list collected again (its largest terms)
constexpr uint32_t kPathSplit = 1u << 17;      // token-only row finished from chunks read by several workgroups
constexpr uint32_t kPathError = 0x80000000u;

// Phase timestamps (measurement builds only, -DLLZ_PHASE_STAMPS): thread 0
// of a row's workgroup records s_memrealtime (100 MHz) at the boundaries of
// the kernel's phases, slot k of row r at llz_phase_stamps[r * kStampSlots +
// k].  In ordinary builds LLZ_STAMP compiles to nothing.
constexpr int kStampRows = 4096;
constexpr int kStampSlots = 60;
#ifdef LLZ_PHASE_STAMPS
static __device__ unsigned long long llz_phase_stamps[kStampRows * kStampSlots];  // read by llz_stats.hip's copy-out
#define LLZ_STAMP(row, k)                                                                     \
  do {                                                                                        \
    if (threadIdx.x == 0 && (row) < ::llz::kStampRows)                                        \
      ::llz::llz_phase_stamps[(row) * ::llz::kStampSlots + (k)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#else
#define LLZ_STAMP(row, k) \
  do {                    \
  } while (0)
#endif

struct RowParams {
  float temperature;
  float top_p;
  float min_p;
  float typical_p;
  uint32_t top_k;
  float cand_theta;   // e >= cand_theta enters the candidate list
  float tok_theta;    // token-only rows: e >= tok_theta enters their list (cand_theta, or 2^-10 without min-p)
  float l2e_t;        // RN(log2(e) / temperature)
  int32_t n;          // vocab
  int32_t rows;
  int32_t kept_cap;
  int64_t src_stride;
  int64_t orig_stride;
  uint32_t flags;
  uint32_t qcap;  // special-queue chunk size override for tests (0: the kernel's own)
  uint32_t xf_src;   // kXf* bits applied to reads of src (the chain's input)
  uint32_t xf_orig;  // kXf* bits applied to reads of orig (sampleArgmax's input)
  float cap;         // final-logit soft-cap s (kXfCap)
  float inv_scale;   // RN(1 / logit_scale) (kXfScale)
  float rpen;        // repetition penalty (kXfPen)
  float rpen_inv;    // RN(1 / rpen): kXmCap's estimate of a penalised logit
  float cap_a2;      // kXmCap: RN(2 log2(e) / cap)
  float cap_c;       // kXmCap: RN(cap * inv_scale), the soft-capped logits' bound
  float est_xe;      // kXmCap: bound of the estimates' relative error beyond the plain rows' (0 otherwise)
  int32_t pen_w;     // kXfPen: window length (<= kPenMax)
  int64_t prev_stride;
  int32_t fb_slots;  // full-row fallback buffers in the workspace
  int32_t grid;      // k_stats workgroups: rows [0, grid) one each, the rest claimed (Q.claim)
  uint64_t epoch;    // this call's tag: a fallback slot whose owner word holds it is in use
  double tok_rs;     // token path: the recursive-summation bound g / (1 - g), g = (n - 1) 2^-24
  double tok_rwk;    // token path: u / (1 - u) (1 + gamma_n) (1 + 2^-9), the weighted bound's factor (0: gamma_n >= 1/2)
  int32_t split_s;   // split rows: chunks per row (0: rows are not split)
  int32_t split_nv;  // split rows: float4 per thread per chunk (chunk = 2048 split_nv logits)
  float split_b;     // split rows: a chunk's elements with (m_c - v) l2e_t < split_b may be candidates
  float split_bs;    // split rows: 256 / split_b (histogram bins per unit of log2)
};

// Split rows: one chunk's summary and the row's record in the workspace
// (words written and read only through device-coherent atomic accesses).
struct SplitRec {
  unsigned long long tag;  // the call's epoch once the words below are final
  unsigned long long mc;   // bits of the chunk's maximum m (NaNs skipped) | bits of c = RN(m l2e_t) << 32
  unsigned long long sv;   // bits of s = sum of exp2(fma(v, l2e_t, -c)) | bits of vt << 32, the largest
                           // logit of the chunk's possible candidates left out of its list (-inf: none)
  unsigned long long nf;   // entries of its list | 0x10000 for a NaN or a maximum beyond 3e38 | bits of the
                           // sum of exp2(fma(v, l2e_t, -c)) (n - pos) << 32
};
struct SplitRow {
  SplitRec rec[kSplitMax];
  unsigned long long elect;  // the call's epoch once a workgroup has taken the row's merge
  unsigned long long pad[7];
  unsigned long long cand[kSplitMax * kSplitK];  // chunk k's list at [k kSplitK, k kSplitK + ncoll): logit bits | position << 32
};

struct RowPtrs {
  const float* src;       // rows the chain reads (penalised copy or the caller's)
  const float* orig;      // the caller's rows (sampleArgmax exits)
  const float* uniforms;  // [rows]
  uint32_t* tokens;
  uint8_t* consumed;
  uint32_t* kept_count;
  uint32_t* kept_ids;
  float* kept_probs;
  float* row_stats;
  uint32_t* status;
  uint64_t* cand;         // [rows][kCandCap] candidate list
  uint32_t* fb;           // 6 x [fb_slots][n] u32 (full-row fallback sort buffers)
  uint8_t* fb_mask;       // [fb_slots][n]
  unsigned long long* fb_owner;  // [fb_slots] epoch of the row using each slot
  uint32_t* qovf;         // [min(rows, kMaxGrid)][kQovfRow] k_stats special-queue overflow, per workgroup
  unsigned long long* claim;  // rows claimed beyond the grid: (epoch tag << 24) | count
  const uint32_t* prev_win;  // kXfPen: row 0's window (its last pen_w history tokens)
  SplitRow* split;           // [rows] split rows' chunk summaries and lists
};

// k_stats's one kernel argument.
struct KArgs {
  RowParams P;
  RowPtrs Q;
};

hipError_t launch_penalty(const float* logits, int64_t stride, int rows, int n, const uint32_t* prev,
                          int n_prev, int64_t prev_stride, int window, float penalty, uint32_t xf, float cap,
                          float inv_scale, float* out, hipStream_t st);
hipError_t launch_argmax(const float* logits, int64_t stride, int rows, int n, uint32_t xf, float cap,
                         float inv_scale, uint32_t* tokens, uint8_t* consumed, uint32_t* kept_count,
                         uint32_t* path, hipStream_t st);
hipError_t launch_sample(const RowParams& P, const RowPtrs& Q, hipEvent_t ev_begin, hipEvent_t ev_end,
                         hipStream_t st);
hipError_t launch_math_probe(const float* in, float* out_exp, float* out_log, float* out_expm1, float* out_tanh,
                             int64_t n, hipStream_t st);
hipError_t launch_hw_error(int op, uint32_t first, uint32_t count, uint32_t* max_err, hipStream_t st);

}  // namespace llz
