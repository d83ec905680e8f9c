// Drives the host code of libllzsample.so's C ABI (llama.zig_amd/csrc/
// llz_api.cpp, compiled with AddressSanitizer and UndefinedBehaviorSanitizer
// for the host only) without a GPU: argument validation, workspace sizing
// and the reference's PRNG.  Exit status 0 = no sanitizer report.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>

#include "../../include/llz_sampler.h"

int main() {
  llz_sampler_config cfg;
  llz_sampler_config_default(&cfg);
  if (cfg.temperature != 0.8f || cfg.repetition_window != 32) return 1;
  // workspace sizes for every shape class, including huge windows
  const int32_t shapes[][2] = {{1, 1}, {1, 128256}, {256, 128256}, {1024, 256000}, {4096, 128256}};
  for (auto& sh : shapes) {
    for (uint32_t win : {0u, 32u, 64u, 65u, 0xffffffffu}) {
      cfg.repetition_window = win;
      cfg.repetition_penalty = 1.3f;
      for (int32_t n_prev : {0, 1, 64, 200}) {
        const size_t b = llz_sample_workspace_bytes(sh[0], sh[1], &cfg, n_prev);
        if (b == 0) return 2;
      }
    }
  }
  if (llz_sample_workspace_bytes(0, 10, &cfg, 0) != 0) return 3;
  // validation returns before any HIP call
  float fake_f = 0.0f;
  uint32_t fake_u = 0;
  char ws[64];
  if (llz_sample_rows(nullptr, 16, 1, 16, &cfg, nullptr, nullptr, 0, 0, &fake_f, &fake_u, nullptr, nullptr, ws,
                      sizeof ws, nullptr) != LLZ_E_INVALID_ARG)
    return 4;
  if (llz_sample_rows(&fake_f, 8, 1, 16, &cfg, nullptr, nullptr, 0, 0, &fake_f, &fake_u, nullptr, nullptr, ws,
                      sizeof ws, nullptr) != LLZ_E_INVALID_ARG)
    return 5;
  cfg.temperature = 1.0f;
  if (llz_sample_rows(&fake_f, 16, 1, 16, &cfg, nullptr, nullptr, 0, 0, &fake_f, &fake_u, nullptr, nullptr, ws,
                      sizeof ws, nullptr) != LLZ_E_WORKSPACE)
    return 6;
  if (llz_argmax_rows(nullptr, 16, 1, 16, nullptr, &fake_u, nullptr) != LLZ_E_INVALID_ARG) return 7;
  for (int c = -6; c <= 0; ++c)
    if (!llz_strerror(c)) return 8;
  // the PRNG: many draws, every value in (0, 1)
  uint64_t st[4];
  llz_rng_seed(st, 0xDEADBEEFull);
  static float u[1 << 16];
  llz_rng_uniforms(st, u, 1 << 16);
  for (float v : u)
    if (!(v > 0.0f && v < 1.0f)) return 9;
  llz_sampler* s = nullptr;
  const int rc = llz_sampler_create(&cfg, 0, &s);  // no GPU here: an error, no leak
  if (rc == LLZ_OK) llz_sampler_destroy(s);
  llz_sampler_destroy(nullptr);
  std::puts("host sanitizer run: ok");
  return 0;
}
