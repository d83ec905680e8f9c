/*
 * llz_oracle.c -- CPU restatement of llama.zig's token sampler (TEST
 * INFRASTRUCTURE ONLY: the shipped library never links or calls it).
 *
 * Third-party algorithms restated below, with the notices their authors ask
 * to be kept:
 *   expf, logf, expm1f (FreeBSD msun e_expf.c, e_logf.c, s_expm1f.c):
 *     Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
 *     Developed at SunPro, a Sun Microsystems, Inc. business.
 *     Permission to use, copy, modify, and distribute this software is
 *     freely granted, provided that this notice is preserved.
 *     (Float versions by Ian Lance Taylor, Cygnus Support.)
 *   tanhf (musl src/math/tanhf.c): musl libc, Copyright (c) 2005-2020 Rich
 *     Felker, et al., MIT license ("The above copyright notice and this
 *     permission notice shall be included in all copies or substantial
 *     portions of the Software").
 *
 * Every function cites the reference line it follows.  The restatement is
 * deliberately literal: sequential f32 loops in the reference's order, a
 * stable sort with the reference's comparator, the same early exits.  Build
 * with -O2 -ffp-contract=off and no fast-math so that every f32 operation
 * rounds exactly once, as in Zig's default (strict) float mode.
 */
#include "llz_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#if defined(__FAST_MATH__)
#error "the oracle must not be built with fast-math"
#endif

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------
 * exp / log for f32.  The sampler calls std.math.exp (sampler.zig:85) and
 * @log (sampler.zig:131,136).  Zig lowers both to its compiler_rt expf/logf,
 * which carry the FreeBSD msun algorithms (e_expf.c, e_logf.c; Sun
 * Microsystems 1993, as shipped in musl <= 1.1.19).  This is a fresh
 * restatement of those published algorithms in the musl control flow.
 * ---------------------------------------------------------------------- */

/* RN(y * 2^k) for finite y (musl scalbnf: two exact power-of-two steps
 * then one rounding multiply). */
static float scale_by_pow2(float y, int k)
{
    if (k > 127) {
        y *= 0x1p127f;
        k -= 127;
        if (k > 127) {
            y *= 0x1p127f;
            k -= 127;
            if (k > 127) k = 127;
        }
    } else if (k < -126) {
        y *= 0x1p-102f;
        k += 102;
        if (k < -126) {
            y *= 0x1p-102f;
            k += 102;
            if (k < -126) k = -126;
        }
    }
    return y * u2f((uint32_t)(0x7f + k) << 23);
}

float llz_oracle_expf(float x)
{
    static const float half[2] = {0.5f, -0.5f};
    const float ln2hi = 6.9314575195e-1f;   /* 0x3f317200 */
    const float ln2lo = 1.4286067653e-6f;   /* 0x35bfbe8e */
    const float invln2 = 1.4426950216e+0f;  /* 0x3fb8aa3b */
    const float P1 = 1.6666625440e-1f;      /* 0xaaaa8f.0p-26 */
    const float P2 = -2.7667332906e-3f;     /* -0xb55215.0p-32 */

    uint32_t hx = f2u(x);
    int sign = (int)(hx >> 31);
    hx &= 0x7fffffffu;

    if (hx >= 0x42aeac50u) {                  /* |x| >= 87.33655 or NaN */
        if (hx > 0x7f800000u) return x;        /* NaN */
        if (hx >= 0x42b17218u && !sign)        /* x >= 88.722839: overflow */
            return x * 0x1p127f;
        if (sign && hx >= 0x42cff1b5u)         /* x <= -103.972084 */
            return 0.0f;
    }

    float hi, lo;
    int k;
    if (hx > 0x3eb17218u) {                   /* |x| > ln2/2 */
        if (hx > 0x3f851592u)                  /* |x| > 3 ln2 / 2 */
            k = (int)(invln2 * x + half[sign]);
        else
            k = 1 - sign - sign;
        hi = x - (float)k * ln2hi;             /* exact */
        lo = (float)k * ln2lo;
        x = hi - lo;
    } else if (hx > 0x39000000u) {            /* |x| > 2^-13 */
        k = 0;
        hi = x;
        lo = 0.0f;
    } else {
        return 1.0f + x;
    }

    float xx = x * x;
    float c = x - xx * (P1 + xx * P2);
    float y = 1.0f + (x * c / (2.0f - c) - lo + hi);
    return k == 0 ? y : scale_by_pow2(y, k);
}

float llz_oracle_logf(float x)
{
    const float ln2_hi = 6.9313812256e-01f; /* 0x3f317180 */
    const float ln2_lo = 9.0580006145e-06f; /* 0x3717f7d1 */
    const float Lg1 = 0xaaaaaa.0p-24f;      /* 0.66666662693 */
    const float Lg2 = 0xccce13.0p-25f;      /* 0.40000972152 */
    const float Lg3 = 0x91e9ee.0p-25f;      /* 0.28498786688 */
    const float Lg4 = 0xf89e26.0p-26f;      /* 0.24279078841 */

    uint32_t ix = f2u(x);
    int k = 0;
    if (ix < 0x00800000u || (ix >> 31)) {   /* x < 2^-126, or negative */
        if ((ix << 1) == 0) return -INFINITY;
        if (ix >> 31) return NAN;
        k -= 25;                             /* subnormal: scale up */
        x *= 0x1p25f;
        ix = f2u(x);
    } else if (ix >= 0x7f800000u) {
        return x;
    } else if (ix == 0x3f800000u) {
        return 0.0f;
    }

    /* reduce x into [sqrt(2)/2, sqrt(2)] */
    ix += 0x3f800000u - 0x3f3504f3u;
    k += (int)(ix >> 23) - 0x7f;
    ix = (ix & 0x007fffffu) + 0x3f3504f3u;
    x = u2f(ix);

    float f = x - 1.0f;
    float s = f / (2.0f + f);
    float z = s * s;
    float w = z * z;
    float t1 = w * (Lg2 + w * Lg4);
    float t2 = z * (Lg1 + w * Lg3);
    float R = t2 + t1;
    float hfsq = 0.5f * f * f;
    float dk = (float)k;
    return s * (hfsq + R) + dk * ln2_lo - hfsq + f + dk * ln2_hi;
}

/* Sensitivity study only (oracle/libm_sensitivity.py): when set, the chain
 * evaluates its exp and log with the C library's expf / logf instead of the
 * msun restatement above, to measure how much an ulp-level difference in
 * Zig's std.math.exp / @log could change kept sets and tokens. */
static int g_use_libm = 0;

void llz_oracle_use_libm(int on) { g_use_libm = on; }

static inline float chain_expf(float x) { return g_use_libm ? expf(x) : llz_oracle_expf(x); }
static inline float chain_logf(float x) { return g_use_libm ? logf(x) : llz_oracle_logf(x); }

void llz_oracle_expf_array(const float *in, float *out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = llz_oracle_expf(in[i]);
}

void llz_oracle_logf_array(const float *in, float *out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = llz_oracle_logf(in[i]);
}

/* ------------------------------------------------------------------------
 * expm1 / tanh for f32.  The reference's decode loop soft-caps the final
 * logits with std.math.tanh (main.zig:653-658) before the sampler sees them.
 * Zig's std.math.tanh / expm1 for f32 are ports of musl's tanhf.c /
 * expm1f.c (musl 1.2.x; expm1f.c derives from FreeBSD msun s_expm1f.c).
 * This is a fresh restatement of those published algorithms.
 * ---------------------------------------------------------------------- */
float llz_oracle_expm1f(float x)
{
    const float o_threshold = 8.8721679688e+01f; /* 0x42b17180 */
    const float ln2_hi = 6.9313812256e-01f;      /* 0x3f317180 */
    const float ln2_lo = 9.0580006145e-06f;      /* 0x3717f7d1 */
    const float invln2 = 1.4426950216e+00f;      /* 0x3fb8aa3b */
    const float Q1 = -3.3333212137e-2f;          /* -0x888868.0p-28 */
    const float Q2 = 1.5807170421e-3f;           /*  0xcf3010.0p-33 */
    const uint32_t ux = f2u(x);
    const uint32_t hx = ux & 0x7fffffffu;
    const int sign = (int)(ux >> 31);
    float hi, lo, c = 0.0f, t, e, hfx, hxs, r1, twopk, y;
    int k;

    if (hx >= 0x4195b844u) {          /* |x| >= 27 ln2, or not finite */
        if (hx > 0x7f800000u) return x; /* NaN */
        if (sign) return -1.0f;
        if (x > o_threshold) return x * 0x1p127f;
    }
    if (hx > 0x3eb17218u) {           /* |x| > ln2 / 2 */
        if (hx < 0x3f851592u) {       /* and |x| < 1.5 ln2 */
            if (!sign) { hi = x - ln2_hi; lo = ln2_lo; k = 1; }
            else { hi = x + ln2_hi; lo = -ln2_lo; k = -1; }
        } else {
            k = (int)(invln2 * x + (sign ? -0.5f : 0.5f));
            t = (float)k;
            hi = x - t * ln2_hi;
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000u) {    /* |x| < 2^-25 */
        return x;
    } else {
        k = 0;
    }
    hfx = 0.5f * x;
    hxs = x * hfx;
    r1 = 1.0f + hxs * (Q1 + hxs * Q2);
    t = 3.0f - r1 * hfx;
    e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = x * (e - c) - c;
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) {
        if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
        return 1.0f + 2.0f * (x - e);
    }
    twopk = u2f((uint32_t)(0x7f + k) << 23);
    if (k < 0 || k > 56) {
        y = x - e + 1.0f;
        if (k == 128) y = y * 2.0f * 0x1p127f;
        else y = y * twopk;
        return y - 1.0f;
    }
    {
        const float tmk = u2f((uint32_t)(0x7f - k) << 23); /* 2^-k */
        if (k < 23) y = (x - e + (1.0f - tmk)) * twopk;
        else y = (x - (e + tmk) + 1.0f) * twopk;
    }
    return y;
}

float llz_oracle_tanhf(float x)
{
    const uint32_t ux = f2u(x);
    const uint32_t w = ux & 0x7fffffffu;
    const int sign = (int)(ux >> 31);
    const float ax = u2f(w);
    float t;

    if (w > 0x3f0c9f54u) {            /* |x| > log(3) / 2, or NaN */
        if (w > 0x41200000u) {        /* |x| > 10 */
            t = 1.0f + 0.0f / ax;
        } else {
            t = llz_oracle_expm1f(2.0f * ax);
            t = 1.0f - 2.0f / (t + 2.0f);
        }
    } else if (w > 0x3e82c578u) {     /* |x| > log(5/3) / 2 */
        t = llz_oracle_expm1f(2.0f * ax);
        t = t / (t + 2.0f);
    } else if (w >= 0x00800000u) {    /* normal */
        t = llz_oracle_expm1f(-2.0f * ax);
        t = -t / (t + 2.0f);
    } else {                          /* subnormal or zero */
        t = ax;
    }
    return sign ? -t : t;
}

void llz_oracle_expm1f_array(const float *in, float *out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = llz_oracle_expm1f(in[i]);
}

void llz_oracle_tanhf_array(const float *in, float *out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = llz_oracle_tanhf(in[i]);
}

/* main.zig:653-666: the decode loop's post-processing of the final logits
 * before Sampler.sample: soft-capping v = tanh(v / s) * s when s > 0, then
 * the logit scale v *= 1 / scale when scale is neither 1 nor 0 (the inverse
 * is one f32 division, main.zig:664).  In place. */
void llz_oracle_logit_post(float *x, int64_t n, float softcap, float logit_scale)
{
    if (softcap > 0.0f)
        for (int64_t i = 0; i < n; ++i) x[i] = llz_oracle_tanhf(x[i] / softcap) * softcap;
    if (logit_scale != 1.0f && logit_scale != 0.0f) {
        const float inv = 1.0f / logit_scale;
        for (int64_t i = 0; i < n; ++i) x[i] *= inv;
    }
}

/* ------------------------------------------------------------------------
 * RNG.  sampler.zig:17,22 use std.Random.DefaultPrng = Xoshiro256, seeded
 * through SplitMix64; sampler.zig:162 draws random.float(f32).
 * ---------------------------------------------------------------------- */

uint64_t llz_oracle_splitmix64_next(uint64_t *state)
{
    uint64_t z = (*state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

void llz_oracle_xoshiro_seed(uint64_t s[4], uint64_t seed)
{
    uint64_t sm = seed;
    for (int i = 0; i < 4; ++i) s[i] = llz_oracle_splitmix64_next(&sm);
}

static inline uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

uint64_t llz_oracle_xoshiro_next(uint64_t s[4])
{
    uint64_t result = rotl64(s[0] + s[3], 23) + s[0];
    uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return result;
}

static inline int clz64(uint64_t x) { return x ? __builtin_clzll(x) : 64; }

/* Random.float(f32): 23 mantissa bits from the low bits of one 64-bit draw,
 * exponent 126 - (leading zeros), extended with further draws when the top
 * 41 bits are all zero.  Random.int(u32) is the low half of one draw. */
float llz_oracle_random_f32(uint64_t s[4])
{
    uint64_t rnd = llz_oracle_xoshiro_next(s);
    int lz = clz64(rnd);
    if (lz >= 41) {
        lz = 41 + clz64(llz_oracle_xoshiro_next(s));
        if (lz == 41 + 64) {
            uint32_t r32 = (uint32_t)llz_oracle_xoshiro_next(s);
            lz += __builtin_clz(r32 | 0x7ffu);
        }
    }
    uint32_t mant = (uint32_t)(rnd & 0x7fffffu);
    uint32_t expo = (uint32_t)(126 - lz) << 23;
    return u2f(expo | mant);
}

void llz_oracle_uniforms(uint64_t s[4], float *out, int64_t count)
{
    for (int64_t i = 0; i < count; ++i) out[i] = llz_oracle_random_f32(s);
}

/* ------------------------------------------------------------------------
 * sampler.zig:31-41 sampleArgmax: first index of the strict running max.
 * ---------------------------------------------------------------------- */
uint32_t llz_oracle_argmax(const float *logits, int64_t n)
{
    int64_t best = 0;
    float max_v = logits[0];
    for (int64_t i = 1; i < n; ++i) {
        if (logits[i] > max_v) {
            max_v = logits[i];
            best = i;
        }
    }
    return (uint32_t)best;
}

/* ------------------------------------------------------------------------
 * Stable merge sort of an index array by a float key.  desc != 0 orders by
 * key[a] > key[b] (sampler.zig:96-100); desc == 0 by key[a] < key[b]
 * (sampler.zig:142-146).  Stability keeps equal keys in index order, as
 * std.mem.sort (a stable block sort) does.
 * ---------------------------------------------------------------------- */
static inline int before(const float *key, uint32_t a, uint32_t b, int desc)
{
    return desc ? (key[a] > key[b]) : (key[a] < key[b]);
}

static void merge_sort(uint32_t *idx, uint32_t *tmp, int64_t n, const float *key, int desc)
{
    /* bottom-up: runs of 16 by insertion sort, then merges */
    const int64_t RUN = 16;
    for (int64_t lo = 0; lo < n; lo += RUN) {
        int64_t hi = lo + RUN < n ? lo + RUN : n;
        for (int64_t i = lo + 1; i < hi; ++i) {
            uint32_t v = idx[i];
            int64_t j = i - 1;
            while (j >= lo && before(key, v, idx[j], desc)) {
                idx[j + 1] = idx[j];
                --j;
            }
            idx[j + 1] = v;
        }
    }
    uint32_t *src = idx, *dst = tmp;
    for (int64_t width = RUN; width < n; width *= 2) {
        for (int64_t lo = 0; lo < n; lo += 2 * width) {
            int64_t mid = lo + width < n ? lo + width : n;
            int64_t hi = lo + 2 * width < n ? lo + 2 * width : n;
            int64_t a = lo, b = mid, o = lo;
            while (a < mid && b < hi) {
                /* take from the right run only if strictly before: stable */
                if (before(key, src[b], src[a], desc)) dst[o++] = src[b++];
                else dst[o++] = src[a++];
            }
            while (a < mid) dst[o++] = src[a++];
            while (b < hi) dst[o++] = src[b++];
        }
        uint32_t *t = src; src = dst; dst = t;
    }
    if (src != idx) memcpy(idx, src, (size_t)n * sizeof(uint32_t));
}

/* ------------------------------------------------------------------------
 * sampler.zig:43-169 sampleWithRandom, with `random.float(f32)` replaced by
 * the argument `u` (consumed only where the reference draws).
 * ---------------------------------------------------------------------- */
static int sample_row_impl(const float *logits, int64_t n, const llz_oracle_cfg *cfg,
                           const uint32_t *prev_tokens, int64_t n_prev, float u,
                           uint64_t *prng, llz_oracle_out *out)
{
    out->consumed = 0;
    out->kept_count = 0;
    out->max_logit = 0.0f;
    out->sum = 0.0f;
    out->entropy = 0.0f;
    out->total = 0.0f;
    out->r0 = 0.0f;
    out->p_max = 0.0f;

    /* :50 */
    if (cfg->temperature <= 0.0f) {
        out->token = llz_oracle_argmax(logits, n);
        out->exit_path = LLZ_EXIT_GREEDY;
        return 0;
    }

    float *penalized = (float *)malloc((size_t)n * sizeof(float));
    float *probs = out->probs ? out->probs : (float *)malloc((size_t)n * sizeof(float));
    uint32_t *indices = out->order ? out->order : (uint32_t *)malloc((size_t)n * sizeof(uint32_t));
    uint32_t *tmp = (uint32_t *)malloc((size_t)n * sizeof(uint32_t));
    uint8_t *selected = out->selected ? out->selected : (uint8_t *)malloc((size_t)n);
    float *dev = NULL;
    uint32_t *typical_order = NULL;
    int rc = 0;
    if (!penalized || !probs || !indices || !tmp || !selected) { rc = -1; goto done; }

    /* :54-75 repetition penalty, literally O(n * window) */
    memcpy(penalized, logits, (size_t)n * sizeof(float));
    if (cfg->repetition_penalty != 1.0f && n_prev > 0) {
        int64_t window = n_prev < (int64_t)cfg->repetition_window ? n_prev
                                                                  : (int64_t)cfg->repetition_window;
        int64_t start = n_prev - window;
        for (int64_t i = 0; i < n; ++i) {
            for (int64_t t = start; t < n_prev; ++t) {
                if ((uint32_t)i == prev_tokens[t]) {
                    if (penalized[i] > 0.0f) penalized[i] /= cfg->repetition_penalty;
                    else penalized[i] *= cfg->repetition_penalty;
                    break;
                }
            }
        }
    }

    /* :80-81 */
    float max_logit = penalized[0];
    for (int64_t i = 1; i < n; ++i) max_logit = fmaxf(max_logit, penalized[i]);
    out->max_logit = max_logit;

    /* :83-88 sequential f32 sum in index order */
    float sum = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        float p = chain_expf((penalized[i] - max_logit) / cfg->temperature);
        probs[i] = p;
        sum += p;
    }
    out->sum = sum;
    /* :89 */
    if (sum <= 0.0f) {
        out->token = llz_oracle_argmax(logits, n);
        out->exit_path = LLZ_EXIT_SUM_LE0;
        goto done;
    }
    /* :90 */
    for (int64_t i = 0; i < n; ++i) probs[i] /= sum;

    /* :92-100 stable sort by probs descending */
    for (int64_t i = 0; i < n; ++i) indices[i] = (uint32_t)i;
    merge_sort(indices, tmp, n, probs, 1);
    out->p_max = probs[indices[0]];

    /* :102-104 */
    memset(selected, 1, (size_t)n);

    /* :106-109 top-k */
    if (cfg->top_k > 0 && (int64_t)cfg->top_k < n) {
        for (int64_t r = (int64_t)cfg->top_k; r < n; ++r) selected[indices[r]] = 0;
    }

    /* :111-118 top-p, sequential cum over selected in sorted order */
    if (cfg->top_p > 0.0f && cfg->top_p < 1.0f) {
        float cum_p = 0.0f;
        for (int64_t r = 0; r < n; ++r) {
            uint32_t idx = indices[r];
            if (!selected[idx]) continue;
            cum_p += probs[idx];
            if (cum_p > cfg->top_p) selected[idx] = 0;
        }
    }

    /* :120-126 min-p against the unfiltered maximum */
    if (cfg->min_p > 0.0f) {
        float max_prob = probs[indices[0]];
        float p_thresh = max_prob * cfg->min_p;
        for (int64_t r = 0; r < n; ++r) {
            uint32_t idx = indices[r];
            if (selected[idx] && probs[idx] < p_thresh) selected[idx] = 0;
        }
    }

    /* :128-154 typical-p */
    if (cfg->typical_p > 0.0f && cfg->typical_p < 1.0f) {
        float entropy = 0.0f;
        for (int64_t i = 0; i < n; ++i) {
            float p = probs[i];
            if (p > 0.0f) entropy -= p * chain_logf(p);
        }
        out->entropy = entropy;
        dev = (float *)malloc((size_t)n * sizeof(float));
        typical_order = (uint32_t *)malloc((size_t)n * sizeof(uint32_t));
        if (!dev || !typical_order) { rc = -1; goto done; }
        for (int64_t i = 0; i < n; ++i) {
            float p = probs[i];
            float surprise = p > 0.0f ? -chain_logf(p) : INFINITY;
            dev[i] = fabsf(surprise - entropy);
        }
        for (int64_t i = 0; i < n; ++i) typical_order[i] = (uint32_t)i;
        merge_sort(typical_order, tmp, n, dev, 0);
        float cum_typ = 0.0f;
        for (int64_t r = 0; r < n; ++r) {
            uint32_t idx = typical_order[r];
            if (!selected[idx]) continue;
            cum_typ += probs[idx];
            if (cum_typ > cfg->typical_p) selected[idx] = 0;
        }
    }

    /* :156-160 */
    float total_selected = 0.0f;
    uint32_t kept = 0;
    for (int64_t r = 0; r < n; ++r) {
        uint32_t idx = indices[r];
        if (selected[idx]) {
            total_selected += probs[idx];
            ++kept;
        }
    }
    out->kept_count = kept;
    out->total = total_selected;
    if (total_selected <= 0.0f) {
        out->token = indices[0];
        out->exit_path = LLZ_EXIT_EMPTY;
        goto done;
    }

    /* :162-168 the only RNG draw, then the walk */
    out->consumed = 1;
    if (prng) u = llz_oracle_random_f32(prng);
    float r = u * total_selected;
    out->r0 = r;
    for (int64_t q = 0; q < n; ++q) {
        uint32_t idx = indices[q];
        if (!selected[idx]) continue;
        r -= probs[idx];
        if (r <= 0.0f) {
            out->token = idx;
            out->exit_path = LLZ_EXIT_DRAW;
            goto done;
        }
    }
    out->token = indices[0];
    out->exit_path = LLZ_EXIT_FALLBACK;

done:
    free(penalized);
    free(tmp);
    free(dev);
    free(typical_order);
    if (!out->probs) free(probs);
    if (!out->order) free(indices);
    if (!out->selected) free(selected);
    return rc;
}

int llz_oracle_sample_row(const float *logits, int64_t n, const llz_oracle_cfg *cfg,
                          const uint32_t *prev_tokens, int64_t n_prev, float u,
                          llz_oracle_out *out)
{
    return sample_row_impl(logits, n, cfg, prev_tokens, n_prev, u, NULL, out);
}

/* ------------------------------------------------------------------------
 * Batched driver (tests, CPU baseline).
 * ---------------------------------------------------------------------- */
typedef struct {
    const float *logits;
    int64_t n, row_stride;
    const llz_oracle_cfg *cfg;
    const uint32_t *prev;
    int64_t n_prev, prev_stride;
    const float *uniforms;
    uint32_t *tokens;
    uint8_t *consumed;
    uint32_t *kept;
    float *stats;
    int64_t row_begin, row_end;
    int rc;
} rows_job;

static void *rows_worker(void *arg)
{
    rows_job *j = (rows_job *)arg;
    for (int64_t r = j->row_begin; r < j->row_end; ++r) {
        llz_oracle_out o;
        memset(&o, 0, sizeof(o));
        const uint32_t *prev = j->prev ? j->prev + r * j->prev_stride : NULL;
        int rc = llz_oracle_sample_row(j->logits + r * j->row_stride, j->n, j->cfg, prev,
                                       j->n_prev, j->uniforms[r], &o);
        if (rc) { j->rc = rc; return NULL; }
        j->tokens[r] = o.token;
        if (j->consumed) j->consumed[r] = (uint8_t)o.consumed;
        if (j->kept) j->kept[r] = o.kept_count;
        if (j->stats) {
            float *st = j->stats + 4 * r;
            st[0] = o.max_logit;
            st[1] = o.sum;
            st[2] = o.entropy;
            st[3] = o.total;
        }
    }
    return NULL;
}

int llz_oracle_sample_rows(const float *logits, int64_t rows, int64_t n, int64_t row_stride,
                           const llz_oracle_cfg *cfg, const uint32_t *prev_tokens,
                           int64_t n_prev, int64_t prev_stride, const float *uniforms,
                           uint32_t *tokens, uint8_t *consumed, uint32_t *kept_count,
                           int threads)
{
    return llz_oracle_sample_rows_stats(logits, rows, n, row_stride, cfg, prev_tokens, n_prev,
                                        prev_stride, uniforms, tokens, consumed, kept_count, NULL,
                                        threads);
}

int llz_oracle_sample_rows_stats(const float *logits, int64_t rows, int64_t n, int64_t row_stride,
                                 const llz_oracle_cfg *cfg, const uint32_t *prev_tokens,
                                 int64_t n_prev, int64_t prev_stride, const float *uniforms,
                                 uint32_t *tokens, uint8_t *consumed, uint32_t *kept_count,
                                 float *stats, int threads)
{
    if (threads < 1) threads = 1;
    if (threads > rows) threads = (int)(rows > 0 ? rows : 1);
    rows_job jobs[256];
    pthread_t tids[256];
    if (threads > 256) threads = 256;
    int64_t per = (rows + threads - 1) / threads;
    for (int t = 0; t < threads; ++t) {
        rows_job *j = &jobs[t];
        j->logits = logits; j->n = n; j->row_stride = row_stride; j->cfg = cfg;
        j->prev = prev_tokens; j->n_prev = n_prev; j->prev_stride = prev_stride;
        j->uniforms = uniforms; j->tokens = tokens; j->consumed = consumed; j->kept = kept_count;
        j->stats = stats;
        j->row_begin = t * per;
        j->row_end = (t + 1) * per < rows ? (t + 1) * per : rows;
        j->rc = 0;
    }
    if (threads == 1) {
        rows_worker(&jobs[0]);
        return jobs[0].rc;
    }
    for (int t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, rows_worker, &jobs[t]);
    int rc = 0;
    for (int t = 0; t < threads; ++t) {
        pthread_join(tids[t], NULL);
        if (jobs[t].rc) rc = jobs[t].rc;
    }
    return rc;
}

/* sampler.zig:19-28: seed fallback, one PRNG stream across calls, the
 * stream advances only when the draw line executes. */
void llz_oracle_sampler_init(llz_oracle_sampler *s, const llz_oracle_cfg *cfg)
{
    s->cfg = *cfg;
    llz_oracle_xoshiro_seed(s->prng, cfg->seed != 0 ? cfg->seed : 0xDEADBEEFull);
}

int llz_oracle_sampler_sample(llz_oracle_sampler *s, const float *logits, int64_t n,
                              const uint32_t *prev_tokens, int64_t n_prev, uint32_t *token)
{
    /* the PRNG is advanced inside, on the draw line only */
    llz_oracle_out o;
    memset(&o, 0, sizeof(o));
    int rc = sample_row_impl(logits, n, &s->cfg, prev_tokens, n_prev, 0.0f, s->prng, &o);
    if (rc) return rc;
    *token = o.token;
    return 0;
}
