/*
 * llz_sampler.h -- C ABI of the MI355X token-sampling library (libllzsample.so).
 *
 * Drop-in replacement for llama.zig's sampler (src/sampler.zig).  The
 * reference's Zig API is
 *     Sampler.init(cfg: SamplerConfig) Sampler                      sampler.zig:19-24
 *     Sampler.sample(self, allocator, logits, prev_tokens) !TokenID sampler.zig:26-28
 *     sampleArgmax(logits) TokenID                                  sampler.zig:31-41
 * and its decode loop calls them at main.zig:508-518 and main.zig:667.
 * This header exposes:
 *   - llz_sample_rows / llz_argmax_rows: batched, device-resident, async on a
 *     HIP stream; the kernels behind them reproduce sampleWithRandom
 *     (sampler.zig:43-169) bit for bit given the same uniform per row;
 *   - llz_sampler_*: a host-side object with the reference's Sampler
 *     semantics (seed fallback, one PRNG stream, a draw consumed only when the
 *     reference draws), for a one-line swap in main.zig;
 *   - llz_rng_*: the reference's PRNG (std.Random.DefaultPrng seeded by
 *     SplitMix64, Random.float(f32)), so callers can generate per-row
 *     uniforms from the same seeded stream.
 *
 * Conventions: plain pointers and sizes; `stream` is a hipStream_t passed as
 * void* (NULL = the default stream); device pointers are marked d_.  Every
 * function returns 0 (LLZ_OK) or a negative LLZ_E* code; llz_strerror names
 * it.  llz_sample_rows and llz_argmax_rows never allocate: the caller passes
 * the workspace sized by llz_sample_workspace_bytes.
 */
#ifndef LLZ_SAMPLER_H
#define LLZ_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    LLZ_OK = 0,
    LLZ_E_INVALID_ARG = -1,   /* null pointer, rows/vocab <= 0, NaN temperature, ... */
    LLZ_E_WORKSPACE = -2,     /* workspace missing or smaller than required          */
    LLZ_E_HIP = -3,           /* a HIP runtime call failed                           */
    LLZ_E_OOM = -4,           /* host-side object could not allocate                 */
    LLZ_E_NO_DEVICE = -5,     /* no usable HIP device                                */
    LLZ_E_SCRATCH = -6        /* llz_sample_rows_noalloc: the call needs more than   */
                              /* its static scratch (LLZ_NOALLOC_SCRATCH_BYTES)      */
};

/* Mirror of SamplerConfig (sampler.zig:4-13).  Field meanings and defaults
 * are the reference's: temperature 0.8, top_k 0, top_p 0.9, min_p 0.0,
 * typical_p 1.0, seed 0 (-> 0xDEADBEEF), repetition_window 32,
 * repetition_penalty 1.1.  A filter is active exactly when the reference's
 * test is true: 0 < top_k < vocab, 0 < top_p < 1, min_p > 0,
 * 0 < typical_p < 1, repetition_penalty != 1 with a non-empty window. */
typedef struct llz_sampler_config {
    float temperature;
    uint32_t top_k;
    float top_p;
    float min_p;
    float typical_p;
    uint32_t reserved;          /* padding before the u64 (an extern struct of the same
                                   fields in the same order has it too); must be 0 */
    uint64_t seed;
    uint32_t repetition_window;
    float repetition_penalty;
} llz_sampler_config;           /* 40 bytes, fields in sampler.zig:4-13's order */

/* Fills `cfg` with SamplerConfig's defaults (sampler.zig:4-13). */
void llz_sampler_config_default(llz_sampler_config *cfg);

/* The decode loop's post-processing of the final logits before the sampler
 * sees them (main.zig:653-666), applied by the kernels as they read each
 * logit (the caller's rows are not written):
 *   final_logit_softcapping > 0:          v = tanh(v / s) * s   (f32 std.math.tanh)
 *   logit_scale != 1 and logit_scale != 0: v = v * RN(1 / logit_scale)
 * A NULL pointer, or {0, 1}, leaves the logits as they are.  Mirrors the
 * model config fields main.zig reads (cfg.final_logit_softcapping,
 * cfg.logit_scale). */
typedef struct llz_logit_post {
    float final_logit_softcapping;
    float logit_scale;
} llz_logit_post;

/* Optional per-row outputs of llz_sample_rows.  Any pointer may be NULL. */
typedef struct llz_sample_extras {
    uint32_t *d_kept_count;     /* [rows] size of the final kept set                        */
    uint32_t *d_kept_ids;       /* [rows][kept_cap] kept ids in (p desc, id asc) order       */
    float *d_kept_probs;        /* [rows][kept_cap] their normalised probabilities          */
    int32_t kept_cap;           /* capacity per row of the two arrays above                 */
    int32_t reserved;
    float *d_row_stats;         /* [rows][4]: max logit, normaliser, entropy, total kept     */
    uint32_t *d_row_path;       /* [rows] the path each row took (LLZ_PATH_* bits)           */
} llz_sample_extras;

/* Bits of d_row_path (diagnostics).  A row with none of the bits 0-7 and 16
 * took the single-pass exact path (the exact normaliser in one read, then the
 * selection on its candidate list).  Bits 8-15 hold a number, not flags: with
 * LLZ_PATH_FULL_SORT set, why the bucket path declined the row (0: it was not
 * tried; 1 .. 255: a reason code of the bucket path, for diagnostics only). */
enum {
    LLZ_PATH_SUM_LE0 = 1,        /* sum <= 0 exit (sampler.zig:89)                         */
    LLZ_PATH_ENTROPY = 2,        /* typical-p entropy pass ran (sampler.zig:128-154)       */
    LLZ_PATH_FULL_SORT = 4,      /* kept set beyond the candidate list: full-row fallback  */
    LLZ_PATH_STREAM_NORM = 8,    /* normaliser not certified in one pass: streaming pass   */
    LLZ_PATH_WALK_ROUNDS = 16,   /* diagnostic: more EXACT segments than one round's slots  */
    LLZ_PATH_RESOLVE_GENERIC = 32, /* diagnostic: a crossing beyond the tabulated binades   */
    LLZ_PATH_BUCKETS = 64,       /* full row without a sort: kept prefix, total, draw from   */
                                 /*   p-key buckets (with LLZ_PATH_FULL_SORT)              */
    LLZ_PATH_TOKEN_ONLY = 128,   /* the token decided without the exact normaliser (calls    */
                                 /*   asking for neither probabilities nor row statistics)  */
    LLZ_PATH_DECLINE_SHIFT = 8,  /* bits 8-15: the bucket path's decline reason (see above)  */
    LLZ_PATH_RECOLLECT = 1 << 16, /* a flooded candidate list collected again, its largest  */
                                 /*   terms only, so the selection ran on a list            */
    LLZ_PATH_SPLIT = 1 << 17,    /* with LLZ_PATH_TOKEN_ONLY: the row was read by several   */
                                 /*   workgroups, one chunk each (calls of few rows)       */
    LLZ_PATH_ERROR = (int)0x80000000u
};

/* Bytes of device workspace llz_sample_rows needs for this shape and
 * configuration (0 on invalid input).  n_prev is the repetition window
 * length per row that will be passed. */
size_t llz_sample_workspace_bytes(int32_t rows, int32_t vocab, const llz_sampler_config *cfg,
                                  int32_t n_prev);

/* Samples one token per row from `rows` fp32 logit rows of length `vocab`
 * (row r at d_logits + r * row_stride), replacing Sampler.sample /
 * sampleWithRandom (sampler.zig:26-28, :43-169) for a batch, after the
 * decode loop's post-processing (main.zig:653-666) given by `post` (may be
 * NULL).  The repetition penalty (sampler.zig:54-75) is applied as the rows
 * are read when the window (min(n_prev, repetition_window)) holds at most 64
 * tokens, else to a penalised copy in the workspace.
 *   d_prev_tokens: repetition history, n_prev ids per row, rows prev_stride
 *                  apart (prev_stride 0 = one history shared by all rows);
 *                  may be NULL when n_prev == 0.
 *   d_uniforms:    [rows] the value random.float(f32) would return at
 *                  sampler.zig:162 for that row.
 *   d_tokens:      [rows] sampled TokenID (sampler.zig's return value).
 *   d_consumed:    [rows] 1 when the row reached the draw (sampler.zig:162)
 *                  and so consumed its uniform, 0 on the early exits
 *                  (temperature <= 0, sum <= 0, empty kept set).  May be NULL.
 * The call is asynchronous on `stream`. */
int llz_sample_rows(const float *d_logits, int64_t row_stride, int32_t rows, int32_t vocab,
                    const llz_sampler_config *cfg, const llz_logit_post *post,
                    const uint32_t *d_prev_tokens, int32_t n_prev,
                    int64_t prev_stride, const float *d_uniforms, uint32_t *d_tokens,
                    uint8_t *d_consumed, const llz_sample_extras *extras, void *d_workspace,
                    size_t workspace_bytes, void *stream);

/* llz_sample_rows without a workspace: the variant for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  It has no counterpart in the reference.
 * The kernels' scratch is a static device array of LLZ_NOALLOC_SCRATCH_BYTES
 * inside the library, one per GPU it runs on, held until the process ends;
 * the call allocates and frees nothing.  A call whose layout does not fit it
 * (llz_sample_workspace_bytes' layout with at most 8 rows' full-row fallback
 * buffers at a time, and no penalised copy beyond the scratch) returns
 * LLZ_E_SCRATCH before any work.  Every call on a GPU shares that GPU's
 * scratch: calls that overlap on one GPU (other streams, other threads) race
 * and must not be issued.  Outputs and semantics are llz_sample_rows'. */
#define LLZ_NOALLOC_SCRATCH_BYTES (96u << 20)
int llz_sample_rows_noalloc(const float *d_logits, int64_t row_stride, int32_t rows, int32_t vocab,
                            const llz_sampler_config *cfg, const llz_logit_post *post,
                            const uint32_t *d_prev_tokens, int32_t n_prev, int64_t prev_stride,
                            const float *d_uniforms, uint32_t *d_tokens, uint8_t *d_consumed,
                            const llz_sample_extras *extras, void *stream);

/* sampleArgmax (sampler.zig:31-41) per row of the post-processed logits
 * (`post` as for llz_sample_rows; may be NULL): the first index of the
 * strict maximum, scanning from index 0.  Replaces the greedy GPU path
 * executeTopK / topk_bda.glsl (compute_graph.zig:948-984, which scales by
 * 1 / logit_scale at topk_bda.glsl:38-40), keeping the reference sampler's
 * tie-break: values that become equal after the scale keep the first index.
 * Asynchronous on `stream`. */
int llz_argmax_rows(const float *d_logits, int64_t row_stride, int32_t rows, int32_t vocab,
                    const llz_logit_post *post, uint32_t *d_tokens, void *stream);

/* ---- the reference's PRNG (std.Random.DefaultPrng, sampler.zig:17,22,162) ---- */

/* state <- Xoshiro256.init(seed): four successive SplitMix64 outputs. */
void llz_rng_seed(uint64_t state[4], uint64_t seed);
/* One xoshiro256++ output. */
uint64_t llz_rng_next(uint64_t state[4]);
/* Random.float(f32). */
float llz_rng_float(uint64_t state[4]);
/* count successive Random.float(f32) draws into out (host memory). */
void llz_rng_uniforms(uint64_t state[4], float *out, int64_t count);

/* ---- host-side Sampler with the reference's lifecycle (sampler.zig:15-28) ---- */

typedef struct llz_sampler llz_sampler;

/* Sampler.init: keeps cfg, seeds the PRNG with seed != 0 ? seed : 0xDEADBEEF.
 * `device` selects the HIP device the sampler runs on. */
int llz_sampler_create(const llz_sampler_config *cfg, int32_t device, llz_sampler **out);
void llz_sampler_destroy(llz_sampler *s);

/* Sampler.sample for one row.  `logits` may be host or device memory
 * (length n); `prev_tokens` is host memory (may be NULL when n_prev == 0).
 * Synchronous: returns after *token is written.  The PRNG advances by one
 * Random.float(f32) only when the row reaches the draw, exactly as
 * sampler.zig:162. */
int llz_sampler_sample(llz_sampler *s, const float *logits, int32_t n,
                       const uint32_t *prev_tokens, int32_t n_prev, uint32_t *token);

/* Sampler.sample for one row with the uniform supplied by the caller: for a
 * caller that keeps the reference's PRNG itself (the Zig binding keeps
 * std.Random.DefaultPrng and draws random.float(f32) before the call).
 * *consumed is 1 when the row reached the draw (sampler.zig:162) and so used
 * u, 0 when it left the chain before it (temperature <= 0, sum <= 0, empty
 * kept set): the caller then undoes its draw.  The sampler's own PRNG is
 * neither used nor advanced.  Synchronous. */
int llz_sampler_sample_uniform(llz_sampler *s, const float *logits, int32_t n,
                               const uint32_t *prev_tokens, int32_t n_prev, float u,
                               uint32_t *token, uint8_t *consumed);

/* The same with the configuration passed per call (the handle's own is
 * neither used nor changed): one handle, and its device buffers and stream,
 * serves samplers of any configuration, so a caller that creates a sampler
 * per request (engine.zig:215) can share one handle per device.  Calls on
 * one handle must not overlap. */
int llz_sampler_sample_config(llz_sampler *s, const llz_sampler_config *cfg, const float *logits,
                              int32_t n, const uint32_t *prev_tokens, int32_t n_prev, float u,
                              uint32_t *token, uint8_t *consumed);

/* PRNG state snapshot / restore (checkpointing a generation). */
void llz_sampler_get_state(const llz_sampler *s, uint64_t state[4]);
void llz_sampler_set_state(llz_sampler *s, const uint64_t state[4]);

/* Test hook (no counterpart in the reference): evaluates the device's f32
 * exp, log, expm1 and tanh -- the functions the kernels use in place of
 * std.math.exp, @log (sampler.zig:85,131,136) and std.math.tanh
 * (main.zig:656) -- on n inputs.  Any output may be NULL.  Used by the
 * parity tests to compare the GPU math with the CPU oracle. */
int llz_debug_math(const float *d_in, float *d_exp, float *d_log, float *d_expm1, float *d_tanh,
                   int64_t n, void *stream);

/* Test hook (no counterpart in the reference): the largest relative error,
 * in units of 2^-23, of the hardware exp2 (op 0), log2 (op 1) or reciprocal
 * (op 2) that the kernels' estimates use, over the `count` floats whose bit
 * patterns start at `first_bits`, against double precision; op 3: the
 * hardware log2's error relative to max(1, |log2 x|).  Writes
 * round-toward-zero(error * 2^20), saturated at 0xffffffff, to *d_max_err
 * (device memory, one u32, overwritten).  The estimates' error bounds assume
 * at most 1 unit (1 ulp) for ops 0-2 on the ranges the kernels evaluate, and
 * at most 32 units for op 3 (the token path's entropy estimate). */
int llz_debug_hw_error(int32_t op, uint32_t first_bits, uint32_t count, uint32_t *d_max_err, void *stream);

/* Measurement hook (no counterpart in the reference): while set, every
 * llz_sample_rows call records `begin_event` right before and `end_event`
 * right after its per-row sampling kernel, on the call's stream (both are
 * hipEvent_t).  NULL, NULL clears.  Process-wide, not thread-safe; times
 * single launches (each pair of events adds a few microseconds of stream
 * time, so throughput runs leave it cleared). */
int llz_debug_kernel_events(void *begin_event, void *end_event);

/* Test hook (no counterpart in the reference): the special-queue chunk of
 * the single-pass statistics (entries per wave and chunk, 1 .. 127) for the
 * following llz_sample_rows calls, so that tests reach the queue's chunks
 * in the workspace on ordinary rows; 0 restores the kernel's own.  Results
 * do not depend on it.  Process-wide. */
int llz_debug_set_queue_cap(uint32_t cap);

/* Test hook (no counterpart in the reference): split rows for the following
 * llz_sample_rows calls (token-only calls of at most 64 plain rows read each
 * row with several workgroups, one chunk of 2048 nv logits each).  mode 0:
 * the library's choice (the smallest nv <= 8 whose workgroups fit the CUs
 * at once); 1: off; 2, 4 or 8: nv at least that.  Results do not depend on
 * it.  Process-wide.  LLZ_E_INVALID_ARG for any other mode. */
int llz_debug_set_split(int32_t mode);

/* Name of a return code. */
const char *llz_strerror(int code);

#ifdef __cplusplus
}
#endif
#endif /* LLZ_SAMPLER_H */
