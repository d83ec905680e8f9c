/* Drives the CPU oracle (oracle/llz_oracle.c) under AddressSanitizer and
 * UndefinedBehaviorSanitizer: every exit of the chain, every filter, the
 * penalty's window edge cases, the post-processing and the RNG, on sizes
 * from 1 to a full vocab.  Exit status 0 = no sanitizer report (the
 * sanitizers abort on the first one). */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../oracle/llz_oracle.h"

static float gauss(uint64_t s[4]) {
    float a = llz_oracle_random_f32(s), b = llz_oracle_random_f32(s);
    return sqrtf(-2.0f * logf(a)) * cosf(6.2831853f * b);
}

static void run(const float *x, int64_t n, llz_oracle_cfg cfg, const uint32_t *prev, int64_t n_prev,
                float u) {
    llz_oracle_out o;
    memset(&o, 0, sizeof o);
    o.probs = malloc((size_t)n * sizeof(float));
    o.order = malloc((size_t)n * sizeof(uint32_t));
    o.selected = malloc((size_t)n);
    if (llz_oracle_sample_row(x, n, &cfg, prev, n_prev, u, &o) != 0) abort();
    if (n > 0 && o.token >= (uint32_t)n) abort();
    free(o.probs);
    free(o.order);
    free(o.selected);
}

int main(void) {
    uint64_t s[4];
    llz_oracle_xoshiro_seed(s, 7);
    const int64_t sizes[] = {1, 2, 3, 7, 64, 1000, 4097, 128256};
    uint32_t prev[80];
    for (int i = 0; i < 80; ++i) prev[i] = (uint32_t)(i * 37 % 5000);
    prev[3] = prev[2];
    prev[5] = 0xffffffffu;  /* an id beyond every vocab */
    for (size_t si = 0; si < sizeof sizes / sizeof sizes[0]; ++si) {
        const int64_t n = sizes[si];
        float *x = malloc((size_t)n * sizeof(float));
        for (int64_t i = 0; i < n; ++i) x[i] = 2.0f * gauss(s);
        const llz_oracle_cfg base = {0.8f, 0, 0.9f, 0.0f, 1.0f, 32, 1.1f, 0, 0};
        llz_oracle_cfg c = base;
        run(x, n, c, prev, 80, 0.37f);                 /* defaults with the penalty */
        c.temperature = 0.0f; run(x, n, c, NULL, 0, 0.5f);
        c = base; c.top_k = 40; c.top_p = 0.95f; c.min_p = 0.05f; run(x, n, c, NULL, 0, 0.9f);
        c = base; c.typical_p = 0.5f; c.top_p = 1.0f; run(x, n, c, NULL, 0, 0.1f);
        c = base; c.repetition_window = 0xffffffffu; run(x, n, c, prev, 80, 0.2f);
        c = base; c.top_p = 1e-7f; run(x, n, c, NULL, 0, 0.99f);  /* empty kept set */
        c = base; c.min_p = 1.5f; c.top_p = 1.0f; run(x, n, c, NULL, 0, 0.5f);
        x[0] = NAN; run(x, n, base, NULL, 0, 0.5f);
        for (int64_t i = 0; i < n; ++i) x[i] = -INFINITY;
        run(x, n, base, NULL, 0, 0.5f);
        for (int64_t i = 0; i < n; ++i) x[i] = 1.0f;  /* all ties */
        run(x, n, base, NULL, 0, 0.5f);
        for (int64_t i = 0; i < n; ++i) x[i] = 30.0f * gauss(s);
        llz_oracle_logit_post(x, n, 30.0f, 0.7f);
        run(x, n, base, prev, 80, 0.6f);
        free(x);
    }
    float f[3] = {0.5f, -20.0f, 1e-40f}, g[3];
    llz_oracle_tanhf_array(f, g, 3);
    llz_oracle_expm1f_array(f, g, 3);
    llz_oracle_expf_array(f, g, 3);
    llz_oracle_logf_array(f, g, 3);
    float us[1000];
    llz_oracle_uniforms(s, us, 1000);
    llz_oracle_sampler sm;
    const llz_oracle_cfg sc = {1.0f, 0, 1.0f, 0.0f, 1.0f, 0, 1.0f, 0, 1234};
    llz_oracle_sampler_init(&sm, &sc);
    const float z[4] = {0, 0, 0, 0};
    uint32_t tok;
    for (int i = 0; i < 16; ++i)
        if (llz_oracle_sampler_sample(&sm, z, 4, NULL, 0, &tok) != 0 || tok > 3) abort();
    puts("oracle sanitizer run: ok");
    return 0;
}
