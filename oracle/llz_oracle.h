/*
 * llz_oracle.h -- CPU restatement of llama.zig's token sampler.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this code.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker (or as the CPU baseline
 * that is timed beside the GPU path).
 *
 * What it restates (paths relative to the reference checkout):
 *   src/sampler.zig:4-13     SamplerConfig            -> llz_oracle_cfg
 *   src/sampler.zig:19-24    Sampler.init             -> llz_oracle_sampler_init
 *   src/sampler.zig:26-28    Sampler.sample           -> llz_oracle_sampler_sample
 *   src/sampler.zig:31-41    sampleArgmax             -> llz_oracle_argmax
 *   src/sampler.zig:43-169   sampleWithRandom         -> llz_oracle_sample_row
 * and the Zig standard-library pieces the sampler calls (Zig >= 0.16, not
 * vendored in the reference, build.zig.zon:28):
 *   std.Random.DefaultPrng  = Xoshiro256 (xoshiro256++, Blackman & Vigna 2018)
 *                             seeded by SplitMix64 (Steele, Lea & Flood 2014)
 *   Random.float(f32)       = 23 random mantissa bits + clz-biased exponent
 *   std.math.exp / @log f32 = the FreeBSD msun e_expf.c / e_logf.c algorithms
 *                             (Sun Microsystems 1993) that musl <= 1.1.19 and
 *                             Zig's compiler_rt carry
 *   std.mem.sort            = a stable sort (any stable sort with the same
 *                             comparator yields the same permutation)
 * Float semantics: strict IEEE binary32, round-to-nearest-even, no FMA
 * contraction, no reassociation (build with -ffp-contract=off, no fast-math).
 */
#ifndef LLZ_ORACLE_H
#define LLZ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/sampler.zig:4-13 (field order and defaults kept). */
typedef struct {
    float temperature;          /* 0.8 */
    uint32_t top_k;             /* 0   */
    float top_p;                /* 0.9 */
    float min_p;                /* 0.0 */
    float typical_p;            /* 1.0 */
    uint32_t repetition_window; /* 32  */
    float repetition_penalty;   /* 1.1 */
    uint32_t _pad;
    uint64_t seed;              /* 0   */
} llz_oracle_cfg;

/* Per-row result of sampleWithRandom plus the internal state the parity
 * tests compare against.  Every pointer field is optional (NULL = skip). */
typedef struct {
    uint32_t token;      /* returned TokenID                                  */
    uint32_t consumed;   /* 1 iff sampler.zig:162 (the RNG draw) executed     */
    uint32_t exit_path;  /* LLZ_EXIT_* below                                  */
    uint32_t kept_count; /* |selected| after every filter                     */
    float max_logit;     /* sampler.zig:80-81                                 */
    float sum;           /* sampler.zig:83-88 (sequential f32)                */
    float entropy;       /* sampler.zig:129-132 (0 if typical disabled)       */
    float total;         /* sampler.zig:156-159                               */
    float r0;            /* u * total (sampler.zig:162), 0 if no draw         */
    float p_max;         /* probs[indices[0]]                                 */
    /* arrays of length n (caller-owned) */
    float *probs;        /* normalised probabilities, index order             */
    uint32_t *order;     /* indices sorted by (p desc, idx asc)               */
    uint8_t *selected;   /* final keep mask, index order                      */
} llz_oracle_out;

enum {
    LLZ_EXIT_GREEDY = 0,    /* temperature <= 0 -> sampleArgmax (sampler.zig:50)  */
    LLZ_EXIT_SUM_LE0 = 1,   /* sum <= 0 -> sampleArgmax (sampler.zig:89)          */
    LLZ_EXIT_EMPTY = 2,     /* total_selected <= 0 -> indices[0] (sampler.zig:160) */
    LLZ_EXIT_DRAW = 3,      /* r <= 0 during the walk (sampler.zig:166)           */
    LLZ_EXIT_FALLBACK = 4   /* walk ended without r <= 0 -> indices[0] (:168)     */
};

/* Zig std restatements. */
float llz_oracle_expf(float x);
float llz_oracle_logf(float x);
/* std.math.expm1 / std.math.tanh for f32 (musl expm1f.c / tanhf.c). */
float llz_oracle_expm1f(float x);
float llz_oracle_tanhf(float x);
/* Element-wise over arrays (parity tests of the device math). */
void llz_oracle_expf_array(const float *in, float *out, int64_t n);
void llz_oracle_logf_array(const float *in, float *out, int64_t n);
void llz_oracle_expm1f_array(const float *in, float *out, int64_t n);
void llz_oracle_tanhf_array(const float *in, float *out, int64_t n);

/* main.zig:653-666, the decode loop's final-logit post-processing before
 * Sampler.sample, in place: v = tanh(v / softcap) * softcap when softcap > 0,
 * then v *= 1 / logit_scale when logit_scale is neither 1 nor 0. */
void llz_oracle_logit_post(float *x, int64_t n, float softcap, float logit_scale);
uint64_t llz_oracle_splitmix64_next(uint64_t *state);
void llz_oracle_xoshiro_seed(uint64_t s[4], uint64_t seed);
uint64_t llz_oracle_xoshiro_next(uint64_t s[4]);
float llz_oracle_random_f32(uint64_t s[4]);
/* Fill `out[0..count)` with successive Random.float(f32) draws. */
void llz_oracle_uniforms(uint64_t s[4], float *out, int64_t count);

/* Sensitivity study only: 1 = the chain uses the C library's expf / logf
 * in place of the msun restatement; 0 (default) = the restatement.
 * Process-wide; set it before sampling. */
void llz_oracle_use_libm(int on);

/* sampler.zig:31-41 */
uint32_t llz_oracle_argmax(const float *logits, int64_t n);

/* sampler.zig:43-169 with the single random draw replaced by `u`.
 * Returns 0 on success, -1 on allocation failure. */
int llz_oracle_sample_row(const float *logits, int64_t n, const llz_oracle_cfg *cfg,
                          const uint32_t *prev_tokens, int64_t n_prev, float u,
                          llz_oracle_out *out);

/* Batched convenience used by tests and the CPU baseline: rows are sampled
 * one after another (row r uses uniforms[r]); `threads` > 1 splits the rows
 * over that many POSIX threads.  prev_tokens rows are `prev_stride` apart
 * (0 = one window shared by every row). */
int llz_oracle_sample_rows(const float *logits, int64_t rows, int64_t n, int64_t row_stride,
                           const llz_oracle_cfg *cfg, const uint32_t *prev_tokens,
                           int64_t n_prev, int64_t prev_stride, const float *uniforms,
                           uint32_t *tokens, uint8_t *consumed, uint32_t *kept_count,
                           int threads);

/* The same, plus per row (when stats is not NULL) the maximum logit, the
 * normaliser, the entropy and the kept total: stats[4 r + 0 .. 3]. */
int llz_oracle_sample_rows_stats(const float *logits, int64_t rows, int64_t n, int64_t row_stride,
                                 const llz_oracle_cfg *cfg, const uint32_t *prev_tokens,
                                 int64_t n_prev, int64_t prev_stride, const float *uniforms,
                                 uint32_t *tokens, uint8_t *consumed, uint32_t *kept_count,
                                 float *stats, int threads);

/* Sampler object with the reference's RNG lifecycle (sampler.zig:15-28). */
typedef struct {
    llz_oracle_cfg cfg;
    uint64_t prng[4];
} llz_oracle_sampler;

void llz_oracle_sampler_init(llz_oracle_sampler *s, const llz_oracle_cfg *cfg);
int llz_oracle_sampler_sample(llz_oracle_sampler *s, const float *logits, int64_t n,
                              const uint32_t *prev_tokens, int64_t n_prev, uint32_t *token);

#ifdef __cplusplus
}
#endif
#endif
