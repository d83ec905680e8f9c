// llz_api.cpp -- C ABI of libllzsample.so (declared in include/llz_sampler.h).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>

#include "../../include/llz_sampler.h"
#include "llz_internal.h"

using namespace llz;

namespace {

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) & ~(kAlign - 1); }

// measurement hook: events recorded around the fused sampling kernel (see llz_debug_kernel_events)
hipEvent_t g_ev_begin = nullptr;
hipEvent_t g_ev_end = nullptr;
// test hook: a smaller special-queue chunk (see llz_debug_set_queue_cap)
std::atomic<uint32_t> g_queue_cap{0u};
// test hook: split rows off, or their smallest chunk width (see llz_debug_set_split)
std::atomic<int> g_split_mode{0};

// With LLZ_DEBUG set in the environment, a HIP error behind an LLZ_E_HIP
// return is printed to stderr (the return code alone does not name it).
void report_hip(const char* where, hipError_t e) {
  static const bool on = std::getenv("LLZ_DEBUG") != nullptr;
  if (on) std::fprintf(stderr, "llz: %s: %s (%d)\n", where, hipGetErrorString(e), (int)e);
}

bool penalty_active(const llz_sampler_config* cfg, int32_t n_prev) {
  return cfg->repetition_penalty != 1.0f && n_prev > 0 && cfg->repetition_window > 0;
}

// sampler.zig:60: window = min(len, repetition_window), taken before any
// narrowing (a u32 window of 2^31 or more means the whole history)
int penalty_window(const llz_sampler_config* cfg, int32_t n_prev) {
  return (int)std::min<uint64_t>((uint64_t)cfg->repetition_window, (uint64_t)n_prev);
}

// The penalty goes to a penalised copy when its window is too long to fuse.
bool penalty_copy(const llz_sampler_config* cfg, int32_t n_prev) {
  return penalty_active(cfg, n_prev) && penalty_window(cfg, n_prev) > kPenMax;
}

// kXf bits of main.zig:653-666's post-processing.
uint32_t post_bits(const llz_logit_post* post) {
  if (!post) return 0u;
  uint32_t b = 0u;
  if (post->final_logit_softcapping > 0.0f) b |= kXfCap;
  if (post->logit_scale != 1.0f && post->logit_scale != 0.0f) b |= kXfScale;
  return b;
}

// Workspace layout of one llz_sample_rows call: per row, its status word and
// candidate list (16 KB); per workgroup of the grid (min(rows, kMaxGrid)),
// a special-queue overflow block (128 KB); per call, a pool of full-row
// fallback buffer sets (25 B per logit each, fb_slots_for) with their owner
// words; the penalised copy only for windows too long to fuse.
struct Layout {
  size_t status, claim, cand, qovf, owner, fb, fb_mask, penal, split, total;
  int fb_slots;
  bool has_penal;
};

float candidate_theta(const llz_sampler_config* cfg, int32_t vocab);

// Full-row fallback buffer sets for a call: a row needs one only when its
// kept set can outgrow the candidate list.  With a min-p of at least 2^-10
// every kept term passes the candidate threshold, so only rows with more
// than kCandCap such terms (near-flat rows) need a set: kFbSlotsLean of them;
// otherwise one per row up to kFbSlots (one per CU: no more rows run at once).
// Rows beyond the pool wait for a set (bounded), so the size affects speed only.
constexpr int kFbSlotsLean = 8;
int fb_slots_for(int32_t rows, int32_t vocab, const llz_sampler_config* cfg, int max_slots) {
  int s = std::min(rows, max_slots);
  if (candidate_theta(cfg, vocab) >= 0x1p-10f) s = std::min(s, kFbSlotsLean);
  return s;
}

Layout layout_of(int32_t rows, int32_t vocab, const llz_sampler_config* cfg, int32_t n_prev,
                 int max_slots = kFbSlots) {
  Layout L{};
  const size_t r = (size_t)rows, n = (size_t)vocab;
  L.fb_slots = fb_slots_for(rows, vocab, cfg, max_slots);
  const size_t ns = (size_t)L.fb_slots;
  size_t off = 0;
  L.status = off;  off = align_up(off + r * sizeof(uint32_t));
  L.claim = off;   off = align_up(off + sizeof(uint64_t));
  L.cand = off;    off = align_up(off + r * (size_t)kCandCap * sizeof(uint64_t));
  L.qovf = off;    off = align_up(off + (size_t)std::min(rows, kMaxGrid) * (size_t)kQovfRow * sizeof(uint32_t));
  L.owner = off;   off = align_up(off + ns * sizeof(uint64_t));
  L.fb = off;      off = align_up(off + 6 * ns * n * sizeof(uint32_t));
  L.fb_mask = off; off = align_up(off + ns * n);
  L.has_penal = penalty_copy(cfg, n_prev);
  L.penal = off;   if (L.has_penal) off = align_up(off + r * n * sizeof(float));
  // last, so that a workspace without it holds every other part at the same
  // offsets: calls of at most kSplitRows rows, the split rows' chunk records
  L.split = off;   if (rows <= kSplitRows) off = align_up(off + r * sizeof(SplitRow));
  L.total = off;
  return L;
}

// Per-call epochs tag the fallback slots a call holds (llz_select.h).  Any
// owner word but the current epoch means free, so a workspace needs no
// clearing; the counter starts at an arbitrary 62-bit value so that stale
// memory is unlikely to hold a live epoch.
std::atomic<uint64_t> g_epoch{0x2d5f7a19c3e4b681ull};

// Candidate threshold on e = exp((v - max) / T).  Every element that can be
// kept must satisfy e >= theta, or the row takes the full fallback.
float candidate_theta(const llz_sampler_config* cfg, int32_t vocab) {
  if (vocab <= kCandCap) return 0.0f;  // the whole row fits the list
  float theta = 0x1p-16f;
  if (cfg->min_p > 0.0f) {
    // p < RN(RN(1/S) * min_p) for every e < min_p * (1 - 2^-20)
    theta = (float)((double)cfg->min_p * (1.0 - 0x1p-20));
    theta = std::nextafter(theta, 0.0f);
  }
  // the row maximum (e == 1) and its probability ties must stay certified
  if (!(theta <= 0.5f)) theta = 0.5f;
  return theta;
}

// The number of CUs of the device a stream runs on (cached per device; the
// last stream's device is remembered per thread, since asking the runtime for
// a stream's device costs more than a launch).
int device_cus(hipStream_t st) {
  static std::atomic<int> cache[64];
  thread_local hipStream_t last_st = nullptr;
  thread_local int last_dev = -1;
  int dev = 0;
  if (st && st == last_st) {
    dev = last_dev;
  } else if (st) {
    if (hipStreamGetDevice(st, &dev) != hipSuccess) return -1;
    last_st = st;
    last_dev = dev;
  } else if (hipGetDevice(&dev) != hipSuccess) {
    return -1;
  }
  if (dev < 0 || dev >= 64) return -1;
  int c = cache[dev].load(std::memory_order_relaxed);
  if (c <= 0) {
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) return -1;
    cache[dev].store(c, std::memory_order_relaxed);
  }
  return c;
}

int check_common(const float* d_logits, int64_t row_stride, int32_t rows, int32_t vocab) {
  if (!d_logits || rows <= 0 || vocab <= 0 || row_stride < vocab) return LLZ_E_INVALID_ARG;
  return LLZ_OK;
}

}  // namespace

extern "C" {

void llz_sampler_config_default(llz_sampler_config* cfg) {
  if (!cfg) return;
  std::memset(cfg, 0, sizeof(*cfg));
  cfg->temperature = 0.8f;
  cfg->top_k = 0;
  cfg->top_p = 0.9f;
  cfg->min_p = 0.0f;
  cfg->typical_p = 1.0f;
  cfg->seed = 0;
  cfg->repetition_window = 32;
  cfg->repetition_penalty = 1.1f;
}

const char* llz_strerror(int code) {
  switch (code) {
    case LLZ_OK: return "ok";
    case LLZ_E_INVALID_ARG: return "invalid argument";
    case LLZ_E_WORKSPACE: return "workspace missing or too small";
    case LLZ_E_HIP: return "HIP runtime error";
    case LLZ_E_OOM: return "out of memory";
    case LLZ_E_NO_DEVICE: return "no HIP device";
    case LLZ_E_SCRATCH: return "input too large for the static scratch of llz_sample_rows_noalloc";
    default: return "unknown error";
  }
}

size_t llz_sample_workspace_bytes(int32_t rows, int32_t vocab, const llz_sampler_config* cfg,
                                  int32_t n_prev) {
  if (!cfg || rows <= 0 || vocab <= 0 || n_prev < 0) return 0;
  return layout_of(rows, vocab, cfg, n_prev).total;
}

int llz_argmax_rows(const float* d_logits, int64_t row_stride, int32_t rows, int32_t vocab,
                    const llz_logit_post* post, uint32_t* d_tokens, void* stream) {
  int rc = check_common(d_logits, row_stride, rows, vocab);
  if (rc) return rc;
  if (!d_tokens) return LLZ_E_INVALID_ARG;
  const uint32_t xb = post_bits(post);
  // main.zig:664: the inverse is one f32 division
  const float inv = (xb & kXfScale) ? 1.0f / post->logit_scale : 1.0f;
  hipError_t e = launch_argmax(d_logits, row_stride, rows, vocab, xb, post ? post->final_logit_softcapping : 0.0f,
                               inv, d_tokens, nullptr, nullptr, nullptr, (hipStream_t)stream);
  return e == hipSuccess ? LLZ_OK : LLZ_E_HIP;
}

}  // extern "C"

// llz_sample_rows on a given workspace holding at most max_slots full-row
// fallback buffer sets (llz_sample_rows: the caller's, kFbSlots;
// llz_sample_rows_noalloc: the library's static scratch, kScratchSlots).
static int sample_rows_impl(const float* d_logits, int64_t row_stride, int32_t rows, int32_t vocab,
                            const llz_sampler_config* cfg, const llz_logit_post* post,
                            const uint32_t* d_prev_tokens, int32_t n_prev, int64_t prev_stride,
                            const float* d_uniforms, uint32_t* d_tokens, uint8_t* d_consumed,
                            const llz_sample_extras* extras, void* d_workspace, size_t workspace_bytes,
                            int max_slots, int too_small_code, void* stream) {
  int rc = check_common(d_logits, row_stride, rows, vocab);
  if (rc) return rc;
  if (!cfg || !d_tokens || n_prev < 0 || prev_stride < 0) return LLZ_E_INVALID_ARG;
  if (cfg->temperature != cfg->temperature) return LLZ_E_INVALID_ARG;  // NaN
  if (n_prev > 0 && !d_prev_tokens) return LLZ_E_INVALID_ARG;
  if (extras && (extras->d_kept_ids || extras->d_kept_probs) && extras->kept_cap <= 0)
    return LLZ_E_INVALID_ARG;
  if (rows > (1 << 24) - 1024) return LLZ_E_INVALID_ARG;  // the row-claim counter's width (rows + grid claims)
  hipStream_t st = (hipStream_t)stream;
  const uint32_t xb = post_bits(post);
  const float cap = (xb & kXfCap) ? post->final_logit_softcapping : 0.0f;
  const float inv = (xb & kXfScale) ? 1.0f / post->logit_scale : 1.0f;  // main.zig:664

  // sampler.zig:50 -- greedy rows never draw
  if (cfg->temperature <= 0.0f) {
    hipError_t e = launch_argmax(d_logits, row_stride, rows, vocab, xb, cap, inv, d_tokens, d_consumed,
                                 extras ? extras->d_kept_count : nullptr, extras ? extras->d_row_path : nullptr,
                                 st);
    return e == hipSuccess ? LLZ_OK : LLZ_E_HIP;
  }
  if (!d_uniforms) return LLZ_E_INVALID_ARG;
  if (penalty_active(cfg, n_prev) && cfg->repetition_penalty != cfg->repetition_penalty)
    return LLZ_E_INVALID_ARG;

  const Layout L = layout_of(rows, vocab, cfg, n_prev, max_slots);
  // a workspace that ends before the split rows' records holds the rest
  if (!d_workspace || workspace_bytes < L.split) return too_small_code;
  const bool split_room = rows <= kSplitRows && workspace_bytes >= L.total;
  char* ws = (char*)d_workspace;

  const float* src = d_logits;
  int64_t src_stride = row_stride;
  uint32_t xf_src = xb;
  const bool pen_on = penalty_active(cfg, n_prev);
  const int window = pen_on ? penalty_window(cfg, n_prev) : 0;
  if (L.has_penal) {
    // a window too long to fuse: the penalised, post-processed copy
    float* pen = (float*)(ws + L.penal);
    hipError_t e = launch_penalty(d_logits, row_stride, rows, vocab, d_prev_tokens, n_prev, prev_stride,
                                  window, cfg->repetition_penalty, xb, cap, inv, pen, st);
    if (e != hipSuccess) return LLZ_E_HIP;
    src = pen;
    src_stride = vocab;
    xf_src = 0u;
  } else if (pen_on) {
    xf_src |= kXfPen;  // fused: applied as each row is read
  }
  const bool vec = ((uintptr_t)src % 16 == 0) && (src_stride % 4 == 0);
  hipError_t e = hipSuccess;

  RowParams P{};
  P.temperature = cfg->temperature;
  P.top_p = cfg->top_p;
  P.min_p = cfg->min_p;
  P.typical_p = cfg->typical_p;
  P.top_k = cfg->top_k;
  P.cand_theta = candidate_theta(cfg, vocab);
  P.l2e_t = (float)(1.4426950408889634 / (double)cfg->temperature);
  P.n = vocab;
  P.rows = rows;
  P.kept_cap = extras ? extras->kept_cap : 0;
  P.src_stride = src_stride;
  P.orig_stride = row_stride;
  // the token alone: no probabilities and no row statistics asked for.  With
  // typical-p, k_stats's token path orders the kept terms by their distance
  // to an interval of the reference's entropy (rows it cannot decide take the
  // exact phases); neither split rows nor soft-capped rows take it with
  // typical-p.  The token path's list
  // holds the terms e >= tok_theta: min-p's candidate threshold when it is at
  // least 2^-10; without min-p (the reference's default chain), 2^-10 with
  // top-p, whose cut must then fall inside the list.  Below 2^-10 the list
  // (every term within 7 nats of the maximum) rarely fits, and a row that does
  // not fit pays for the attempt
  const bool tok_minp = P.cand_theta >= 0x1p-10f;
  const bool tok_topp = !tok_minp && !(cfg->min_p > 0.0f) && cfg->top_p > 0.0f && cfg->top_p < 1.0f &&
                        vocab > kCandCap;
  P.tok_theta = tok_minp ? P.cand_theta : (tok_topp ? 0x1p-10f : 0.0f);
  {
    // the token path's interval of S: the factors that depend on n alone
    // (IEEE double, the same values the device would compute)
    const double g1 = (double)(vocab - 1) * 0x1p-24, gn = (double)vocab * 0x1p-24;
    P.tok_rs = g1 / (1.0 - g1);
    P.tok_rwk = gn < 0.5 ? 0x1p-24 / (1.0 - 0x1p-24) * (1.0 + gn / (1.0 - gn)) * (1.0 + 0x1p-9) : 0.0;
  }
  const bool typical_on = cfg->typical_p > 0.0f && cfg->typical_p < 1.0f;
  const bool tok_only = !(extras && (extras->d_kept_probs || extras->d_row_stats)) && (tok_minp || tok_topp) &&
                        !(typical_on && (xf_src & kXfCap));
  P.flags = (cfg->temperature == 1.0f ? kFlagTIsOne : 0u) | (vec ? kFlagVecSrc : 0u) | kFlagFallback |
            (tok_only ? kFlagTokenOnly : 0u);
  P.xf_src = xf_src;
  P.xf_orig = xb;
  P.cap = cap;
  P.inv_scale = inv;
  P.rpen = cfg->repetition_penalty;
  P.rpen_inv = 1.0f / cfg->repetition_penalty;
  P.pen_w = (xf_src & kXfPen) ? window : 0;
  if (xf_src & kXfCap) {
    // soft-capping: k_stats estimates the capped logits from a closed form
    // (cap_est, llz_xform.h) within 20 C 2^-24 of the reference's values (C =
    // cap inv_scale), max(1, rp, 1/rp) 44 C 2^-24 at penalised positions; the
    // estimates' relative error grows by est_xe = l2e_t times that (|C| for
    // a negative logit scale).  Rows with est_xe above 2^-11 (the candidate
    // margins' budget: 2^-16 + est_xe within the 2^-10 of the thresholds),
    // or with parameters outside the bound's assumptions, take the exact
    // streaming path.
    const double C = (double)cap * (double)inv;
    const bool pen = (xf_src & kXfPen) != 0u;
    const double rp = pen ? (double)cfg->repetition_penalty : 1.0;
    const double bound = (pen ? std::max(1.0, std::max(rp, 1.0 / rp)) * 44.0 : 20.0) * std::fabs(C) * 0x1p-24;
    const double xe = (double)P.l2e_t * bound * (1.0 + 0x1p-20);
    const bool ok = cap > 0.0f && std::isfinite(cap) && inv != 0.0f && std::isfinite(inv) && std::fabs(C) < 1.0e30 &&
                    rp > 0.0 && std::isfinite(rp) && P.l2e_t > 0.0f && std::isfinite(P.l2e_t) && xe <= 0x1p-11;
    P.cap_a2 = (float)(2.0 * 1.4426950408889634 / (double)cap);
    P.cap_c = (float)C;
    if (ok)
      P.est_xe = (float)xe;
    else
      P.flags |= kFlagXfExact;
  }
  P.prev_stride = prev_stride;
  P.fb_slots = L.fb_slots;
  {
    // at most one k_stats workgroup per CU (its shared memory allows no more),
    // all resident at once; rows beyond them are claimed
    const int cus = device_cus(st);
    if (cus <= 0) return LLZ_E_HIP;
    P.grid = std::min(std::min(rows, cus), kMaxGrid);
  }
  // Split rows: a token-only call of at most kSplitRows plain, 16-byte
  // aligned rows reads each row with S workgroups of one chunk each (the
  // smallest chunk, 2048 nv logits, whose rows x S workgroups fit the CUs at
  // once), where one workgroup per row would leave most CUs idle.
  // Rows read through post-processing or the fused penalty take chunks of at
  // most 2 float4 per thread: each logit's exact transform is then a few per
  // thread (calls of up to 8 rows at 128k vocab).
  if (split_room && tok_only && !typical_on && vec && vocab % 4 == 0 && P.tok_theta > 0.0f && P.l2e_t > 0.0f &&
      P.l2e_t <= 0x1p40f && g_split_mode.load(std::memory_order_relaxed) != 1) {
    const int cus = device_cus(st);
    const int nv_max = (xf_src | xb) != 0u ? 2 : kSplitNV;
    for (int nv = std::max(1, g_split_mode.load(std::memory_order_relaxed)); nv <= nv_max && cus > 0; nv *= 2) {
      const int s = (vocab + 2048 * nv - 1) / (2048 * nv);
      if (s <= kSplitMax && rows * s <= cus) {
        if (s >= 2) {
          P.split_s = s;
          P.split_nv = nv;
        }
        break;
      }
    }
    // a chunk's possible candidates: d2 = (m_c - v) l2e_t < log2(1 / theta)
    // + 2^-8 (rounded up to a float)
    const double b = std::log2(1.0 / (double)P.tok_theta) + 0x1p-8;
    float bf = (float)b;
    if ((double)bf < b) bf = std::nextafter(bf, INFINITY);
    P.split_b = bf;
    P.split_bs = 256.0f / bf;
  }
  P.epoch = g_epoch.fetch_add(1, std::memory_order_relaxed) & ((1ull << 62) - 1);
  // the test hook's special-queue chunk (0: the kernel's own)
  P.qcap = g_queue_cap.load(std::memory_order_relaxed);

  RowPtrs Q{};
  Q.src = src;
  Q.orig = d_logits;
  Q.uniforms = d_uniforms;
  Q.tokens = d_tokens;
  Q.consumed = d_consumed;
  if (extras) {
    Q.kept_count = extras->d_kept_count;
    Q.kept_ids = extras->d_kept_ids;
    Q.kept_probs = extras->d_kept_probs;
    Q.row_stats = extras->d_row_stats;
  }
  Q.status = (extras && extras->d_row_path) ? extras->d_row_path : (uint32_t*)(ws + L.status);
  Q.cand = (uint64_t*)(ws + L.cand);
  Q.fb = (uint32_t*)(ws + L.fb);
  Q.fb_mask = (uint8_t*)(ws + L.fb_mask);
  Q.fb_owner = (unsigned long long*)(ws + L.owner);
  Q.qovf = (uint32_t*)(ws + L.qovf);
  Q.claim = (unsigned long long*)(ws + L.claim);
  Q.prev_win = (xf_src & kXfPen) ? d_prev_tokens + (n_prev - window) : nullptr;
  Q.split = P.split_s > 0 ? (SplitRow*)(ws + L.split) : nullptr;
  e = launch_sample(P, Q, g_ev_begin, g_ev_end, st);
  if (e != hipSuccess) report_hip("llz_sample_rows: launch", e);
  return e == hipSuccess ? LLZ_OK : LLZ_E_HIP;
}

// ---------------------------------------------------------------------------
// llz_sample_rows_noalloc: the same call on the library's static scratch.
// `scratch` is a host-side stand-in for the device array: host code uses the
// per-device address hipGetSymbolAddress returns for it, never the name.
// Nothing in it needs clearing between calls: the status words, candidate
// lists and queue overflow are written before they are read within a call,
// a fallback slot is free for a call whenever its owner word holds anything
// but that call's epoch, and a split row's chunk records count for a call
// only once tagged with its epoch.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = (size_t)LLZ_NOALLOC_SCRATCH_BYTES;
constexpr int kScratchSlots = 8;  // full-row fallback buffer sets in the scratch
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // per device: the address of its copy of `scratch`

// The scratch of device `dev`, looked up once per device with that device
// current (each GPU holds its own copy of the array at its own address).
int scratch_of(int dev, void** out) {
  if (dev < 0 || dev >= kMaxDevices) return LLZ_E_NO_DEVICE;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) return LLZ_E_HIP;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return LLZ_E_HIP;
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || !ptr) {
      (void)hipGetLastError();
      return LLZ_E_HIP;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return LLZ_OK;
}
}  // namespace

extern "C" {

int llz_sample_rows_noalloc(const float* d_logits, int64_t row_stride, int32_t rows, int32_t vocab,
                            const llz_sampler_config* cfg, const llz_logit_post* post,
                            const uint32_t* d_prev_tokens, int32_t n_prev, int64_t prev_stride,
                            const float* d_uniforms, uint32_t* d_tokens, uint8_t* d_consumed,
                            const llz_sample_extras* extras, void* stream) {
  int rc = check_common(d_logits, row_stride, rows, vocab);
  if (rc) return rc;
  // the device the call's stream runs on
  int dev = 0;
  if (stream) {
    if (hipStreamGetDevice((hipStream_t)stream, &dev) != hipSuccess) return LLZ_E_HIP;
  } else if (hipGetDevice(&dev) != hipSuccess) {
    return LLZ_E_HIP;
  }
  void* ws = nullptr;
  rc = scratch_of(dev, &ws);
  if (rc) return rc;
  return sample_rows_impl(d_logits, row_stride, rows, vocab, cfg, post, d_prev_tokens, n_prev, prev_stride,
                          d_uniforms, d_tokens, d_consumed, extras, ws, kScratchBytes, kScratchSlots,
                          LLZ_E_SCRATCH, stream);
}

int llz_sample_rows(const float* d_logits, int64_t row_stride, int32_t rows, int32_t vocab,
                    const llz_sampler_config* cfg, const llz_logit_post* post,
                    const uint32_t* d_prev_tokens, int32_t n_prev,
                    int64_t prev_stride, const float* d_uniforms, uint32_t* d_tokens,
                    uint8_t* d_consumed, const llz_sample_extras* extras, void* d_workspace,
                    size_t workspace_bytes, void* stream) {
  return sample_rows_impl(d_logits, row_stride, rows, vocab, cfg, post, d_prev_tokens, n_prev, prev_stride,
                          d_uniforms, d_tokens, d_consumed, extras, d_workspace, workspace_bytes, kFbSlots,
                          LLZ_E_WORKSPACE, stream);
}

int llz_debug_set_queue_cap(uint32_t cap) {
  g_queue_cap.store(cap, std::memory_order_relaxed);
  return LLZ_OK;
}

int llz_debug_set_split(int32_t mode) {
  if (!(mode == 0 || mode == 1 || mode == 2 || mode == 4 || mode == 8)) return LLZ_E_INVALID_ARG;
  g_split_mode.store(mode, std::memory_order_relaxed);
  return LLZ_OK;
}

int llz_debug_kernel_events(void* begin_event, void* end_event) {
  g_ev_begin = (hipEvent_t)begin_event;
  g_ev_end = (hipEvent_t)end_event;
  return LLZ_OK;
}

int llz_debug_math(const float* d_in, float* d_exp, float* d_log, float* d_expm1, float* d_tanh, int64_t n,
                   void* stream) {
  if (!d_in || n < 0 || n > ((int64_t)1 << 40)) return LLZ_E_INVALID_ARG;
  if (n == 0) return LLZ_OK;
  hipError_t e = launch_math_probe(d_in, d_exp, d_log, d_expm1, d_tanh, n, (hipStream_t)stream);
  return e == hipSuccess ? LLZ_OK : LLZ_E_HIP;
}

int llz_debug_hw_error(int32_t op, uint32_t first_bits, uint32_t count, uint32_t* d_max_err, void* stream) {
  if (!d_max_err || op < 0 || op > 3 || count == 0) return LLZ_E_INVALID_ARG;
  hipError_t e = launch_hw_error(op, first_bits, count, d_max_err, (hipStream_t)stream);
  return e == hipSuccess ? LLZ_OK : LLZ_E_HIP;
}

// ---------------------------------------------------------------------------
// The reference's PRNG: std.Random.DefaultPrng (xoshiro256++) seeded through
// SplitMix64, and Random.float(f32) (sampler.zig:17,22,162).
// ---------------------------------------------------------------------------
static uint64_t splitmix_next(uint64_t& x) {
  x += 0x9e3779b97f4a7c15ull;
  uint64_t z = x;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

void llz_rng_seed(uint64_t state[4], uint64_t seed) {
  uint64_t x = seed;
  for (int i = 0; i < 4; ++i) state[i] = splitmix_next(x);
}

uint64_t llz_rng_next(uint64_t state[4]) {
  auto rotl = [](uint64_t v, int k) { return (v << k) | (v >> (64 - k)); };
  const uint64_t out = rotl(state[0] + state[3], 23) + state[0];
  const uint64_t t = state[1] << 17;
  state[2] ^= state[0];
  state[3] ^= state[1];
  state[1] ^= state[2];
  state[0] ^= state[3];
  state[2] ^= t;
  state[3] = rotl(state[3], 45);
  return out;
}

float llz_rng_float(uint64_t state[4]) {
  // 23 uniform mantissa bits; exponent from the count of leading zero bits
  // of the same draw (extended with further draws when 41 or more are zero)
  const uint64_t r = llz_rng_next(state);
  int lz = r ? __builtin_clzll(r) : 64;
  if (lz >= 41) {
    const uint64_t r2 = llz_rng_next(state);
    lz = 41 + (r2 ? __builtin_clzll(r2) : 64);
    if (lz == 41 + 64) lz += __builtin_clz((uint32_t)llz_rng_next(state) | 0x7ffu);
  }
  const uint32_t bits = ((uint32_t)(126 - lz) << 23) | (uint32_t)(r & 0x7fffffu);
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

void llz_rng_uniforms(uint64_t state[4], float* out, int64_t count) {
  for (int64_t i = 0; i < count; ++i) out[i] = llz_rng_float(state);
}

// ---------------------------------------------------------------------------
// Host-side Sampler (sampler.zig:15-28).
// ---------------------------------------------------------------------------
struct llz_sampler {
  llz_sampler_config cfg;
  uint64_t prng[4];
  int device;
  hipStream_t stream;
  int32_t cap_n;       // capacity (vocab) of the buffers below
  int32_t cap_prev;
  float* d_logits;     // staging for host logits
  uint32_t* d_prev;
  float* d_u;
  uint32_t* d_token;
  uint8_t* d_consumed;
  void* d_ws;
  size_t ws_bytes;
};

static void sampler_free_buffers(llz_sampler* s) {
  (void)hipFree(s->d_logits);
  (void)hipFree(s->d_prev);
  (void)hipFree(s->d_u);
  (void)hipFree(s->d_token);
  (void)hipFree(s->d_consumed);
  (void)hipFree(s->d_ws);
  s->d_logits = nullptr; s->d_prev = nullptr; s->d_u = nullptr; s->d_token = nullptr;
  s->d_consumed = nullptr; s->d_ws = nullptr; s->ws_bytes = 0; s->cap_n = 0; s->cap_prev = 0;
}

int llz_sampler_create(const llz_sampler_config* cfg, int32_t device, llz_sampler** out) {
  if (!cfg || !out) return LLZ_E_INVALID_ARG;
  if (cfg->temperature != cfg->temperature) return LLZ_E_INVALID_ARG;
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) {
    (void)hipGetLastError();
    return LLZ_E_NO_DEVICE;
  }
  if (device < 0 || device >= ndev) return LLZ_E_INVALID_ARG;
  llz_sampler* s = new (std::nothrow) llz_sampler();
  if (!s) return LLZ_E_OOM;
  s->cfg = *cfg;
  llz_rng_seed(s->prng, cfg->seed != 0 ? cfg->seed : 0xDEADBEEFull);
  s->device = device;
  if (hipSetDevice(device) != hipSuccess || hipStreamCreate(&s->stream) != hipSuccess) {
    delete s;
    return LLZ_E_HIP;
  }
  *out = s;
  return LLZ_OK;
}

void llz_sampler_destroy(llz_sampler* s) {
  if (!s) return;
  (void)hipSetDevice(s->device);
  sampler_free_buffers(s);
  (void)hipStreamDestroy(s->stream);
  delete s;
}

void llz_sampler_get_state(const llz_sampler* s, uint64_t state[4]) {
  if (s && state) std::memcpy(state, s->prng, sizeof(s->prng));
}

void llz_sampler_set_state(llz_sampler* s, const uint64_t state[4]) {
  if (s && state) std::memcpy(s->prng, state, sizeof(s->prng));
}

static bool is_device_ptr(const void* p) {
  hipPointerAttribute_t a;
  if (hipPointerGetAttributes(&a, p) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return a.type == hipMemoryTypeDevice;
}

// One row through llz_sample_rows with the caller's uniform: token and the
// consumed-draw flag (sampler.zig:162 reached).  Synchronous.
static int sampler_run(llz_sampler* s, const llz_sampler_config* cfg, const float* logits, int32_t n,
                       const uint32_t* prev_tokens, int32_t n_prev, float u, uint32_t* token, uint8_t* consumed) {
  if (!s || !cfg || !logits || n <= 0 || !token || n_prev < 0 || (n_prev > 0 && !prev_tokens))
    return LLZ_E_INVALID_ARG;
  if (cfg->temperature != cfg->temperature) return LLZ_E_INVALID_ARG;
  if (hipSetDevice(s->device) != hipSuccess) return LLZ_E_HIP;
  const size_t need_ws = llz_sample_workspace_bytes(1, n, cfg, n_prev);
  if (n > s->cap_n || n_prev > s->cap_prev || need_ws > s->ws_bytes) {
    sampler_free_buffers(s);
    const int32_t cn = n, cp = n_prev > 0 ? n_prev : 1;
    if (hipMalloc(&s->d_logits, (size_t)cn * sizeof(float)) != hipSuccess ||
        hipMalloc(&s->d_prev, (size_t)cp * sizeof(uint32_t)) != hipSuccess ||
        hipMalloc(&s->d_u, sizeof(float)) != hipSuccess ||
        hipMalloc(&s->d_token, sizeof(uint32_t)) != hipSuccess ||
        hipMalloc(&s->d_consumed, 1) != hipSuccess ||
        hipMalloc(&s->d_ws, need_ws) != hipSuccess) {
      sampler_free_buffers(s);
      return LLZ_E_OOM;
    }
    s->cap_n = cn;
    s->cap_prev = cp;
    s->ws_bytes = need_ws;
  }
  const float* d_in = logits;
  if (!is_device_ptr(logits)) {
    if (hipMemcpyAsync(s->d_logits, logits, (size_t)n * sizeof(float), hipMemcpyHostToDevice,
                       s->stream) != hipSuccess)
      return LLZ_E_HIP;
    d_in = s->d_logits;
  }
  if (n_prev > 0 && hipMemcpyAsync(s->d_prev, prev_tokens, (size_t)n_prev * sizeof(uint32_t),
                                   hipMemcpyHostToDevice, s->stream) != hipSuccess)
    return LLZ_E_HIP;
  if (hipMemcpyAsync(s->d_u, &u, sizeof(float), hipMemcpyHostToDevice, s->stream) != hipSuccess)
    return LLZ_E_HIP;
  int rc = llz_sample_rows(d_in, n, 1, n, cfg, nullptr, n_prev > 0 ? s->d_prev : nullptr, n_prev, 0,
                           s->d_u, s->d_token, s->d_consumed, nullptr, s->d_ws, s->ws_bytes,
                           s->stream);
  if (rc != LLZ_OK) return rc;
  uint32_t tok = 0;
  uint8_t con = 0;
  if (hipMemcpyAsync(&tok, s->d_token, sizeof(tok), hipMemcpyDeviceToHost, s->stream) != hipSuccess ||
      hipMemcpyAsync(&con, s->d_consumed, 1, hipMemcpyDeviceToHost, s->stream) != hipSuccess ||
      hipStreamSynchronize(s->stream) != hipSuccess)
    return LLZ_E_HIP;
  *token = tok;
  *consumed = (con != 0 && cfg->temperature > 0.0f) ? 1 : 0;
  return LLZ_OK;
}

int llz_sampler_sample(llz_sampler* s, const float* logits, int32_t n, const uint32_t* prev_tokens,
                       int32_t n_prev, uint32_t* token) {
  if (!s) return LLZ_E_INVALID_ARG;
  // draw as if the row reached sampler.zig:162; undo it if it did not
  uint64_t snap[4];
  std::memcpy(snap, s->prng, sizeof(snap));
  const float u = llz_rng_float(s->prng);
  uint8_t consumed = 0;
  const int rc = sampler_run(s, &s->cfg, logits, n, prev_tokens, n_prev, u, token, &consumed);
  if (rc != LLZ_OK || !consumed) std::memcpy(s->prng, snap, sizeof(snap));
  return rc;
}

int llz_sampler_sample_uniform(llz_sampler* s, const float* logits, int32_t n, const uint32_t* prev_tokens,
                               int32_t n_prev, float u, uint32_t* token, uint8_t* consumed) {
  if (!consumed) return LLZ_E_INVALID_ARG;
  *consumed = 0;
  return s ? sampler_run(s, &s->cfg, logits, n, prev_tokens, n_prev, u, token, consumed) : LLZ_E_INVALID_ARG;
}

int llz_sampler_sample_config(llz_sampler* s, const llz_sampler_config* cfg, const float* logits, int32_t n,
                              const uint32_t* prev_tokens, int32_t n_prev, float u, uint32_t* token,
                              uint8_t* consumed) {
  if (!consumed) return LLZ_E_INVALID_ARG;
  *consumed = 0;
  return sampler_run(s, cfg, logits, n, prev_tokens, n_prev, u, token, consumed);
}

}  // extern "C"
