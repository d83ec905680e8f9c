// llz_kernels.hip -- MI355X (gfx950) kernels around the fused sampling kernel
// (llz_stats.hip):
//   k_penalty     (optional) penalised copy of the rows   sampler.zig:54-75
//   k_math_probe  the device exp/log/expm1/tanh (parity tests)
//   k_argmax      greedy rows (temperature <= 0)          sampler.zig:31-41,50
#include <hip/hip_runtime.h>

#include <algorithm>

#include "llz_internal.h"
#include "llz_rowops.h"

namespace llz {

constexpr int kMaxNT = 256;        // threads of the k_penalty workgroups
constexpr int kMaxPerThread = 16;  // logits per thread in k_penalty

// ---------------------------------------------------------------------------
// k_penalty: penalised copy (sampler.zig:54-75) of the post-processed rows
// (main.zig:653-666), for windows longer than the fused penalty takes.
// Each index is penalised at most once even when it repeats in the window
// (the reference breaks out of the window scan at the first match).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kMaxNT) void k_penalty(const float* __restrict__ logits, int64_t stride,
                                                    int n, const uint32_t* __restrict__ prev,
                                                    int n_prev, int64_t prev_stride, int window,
                                                    float penalty, uint32_t xf, float cap, float inv_scale,
                                                    float* __restrict__ out) {
  const int row = blockIdx.y;
  const int seg0 = blockIdx.x * (kMaxNT * kMaxPerThread);
  const int seg1 = min(n, seg0 + kMaxNT * kMaxPerThread);
  const float* x = logits + (int64_t)row * stride;
  float* y = out + (int64_t)row * n;
  for (int i = seg0 + (int)threadIdx.x; i < seg1; i += kMaxNT) y[i] = logit_post(x[i], xf, cap, inv_scale);
  __syncthreads();
  const uint32_t* pv = prev + (int64_t)row * prev_stride;
  const int w = min(n_prev, window);
  const int start = n_prev - w;
  for (int a = start + (int)threadIdx.x; a < n_prev; a += kMaxNT) {
    const uint32_t tok = pv[a];
    if (tok >= (uint32_t)seg0 && tok < (uint32_t)seg1) {
      bool first = true;
      for (int b = start; b < a; ++b) first = first && (pv[b] != tok);
      if (first) {
        y[tok] = penalise(logit_post(x[tok], xf, cap, inv_scale), penalty);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// k_argmax: one workgroup per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kNT) void k_argmax(const float* __restrict__ logits, int64_t stride,
                                                int n, uint32_t xf, float cap, float inv_scale,
                                                uint32_t* __restrict__ tokens,
                                                uint8_t* __restrict__ consumed,
                                                uint32_t* __restrict__ kept_count,
                                                uint32_t* __restrict__ path) {
  __shared__ WgScratch<kNT> sh;
  int bank = 0;
  const int row = blockIdx.x;
  const RowSrc x{logits + (int64_t)row * stride, xf & ~kXfPen, cap, inv_scale, 1.0f, nullptr};
  const uint32_t tok = wg_argmax_row<kNT>(x, n, sh, bank);
  if (threadIdx.x == 0) {
    tokens[row] = tok;
    if (consumed) consumed[row] = 0;
    if (kept_count) kept_count[row] = 0;
    if (path) path[row] = 0;
  }
}

// ---------------------------------------------------------------------------
// k_math_probe: the device exp/log/expm1/tanh on an array (parity tests of
// the math).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_math_probe(const float* __restrict__ in, float* __restrict__ out_exp,
                                                   float* __restrict__ out_log, float* __restrict__ out_expm1,
                                                   float* __restrict__ out_tanh, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) {
    const float x = in[i];
    if (out_exp) out_exp[i] = exp_f32(x);
    if (out_log) out_log[i] = log_f32(x);
    if (out_expm1) out_expm1[i] = expm1_f32(x);
    if (out_tanh) out_tanh[i] = tanh_f32(x);
  }
}

// ---------------------------------------------------------------------------
// k_hw_error: the largest relative error of the hardware exp2 (op 0), log2
// (op 1) or reciprocal (op 2) over a range of float bit patterns, against
// double precision, as error * 2^43 (units of 2^-23, times 2^20) folded into
// *max_err; op 3: the log2's error relative to max(1, |log2 x|).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_hw_error(int op, uint32_t first, uint32_t count,
                                                  uint32_t* __restrict__ max_err) {
  uint32_t worst = 0;
  const uint64_t step = (uint64_t)gridDim.x * 256u;
  for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < count; i += step) {
    const float x = __uint_as_float(first + (uint32_t)i);
    float r;
    double y;
    if (op == 0) {
      r = __builtin_amdgcn_exp2f(x);
      y = exp2((double)x);
    } else if (op == 1 || op == 3) {
      r = __builtin_amdgcn_logf(x);
      y = log2((double)x);
    } else {
      r = __builtin_amdgcn_rcpf(x);
      y = 1.0 / (double)x;
    }
    const double q = fabs((double)r - y) / (op == 3 ? fmax(1.0, fabs(y)) : fabs(y)) * 0x1p43;
    worst = max(worst, q < 4.0e9 ? (uint32_t)q : 0xffffffffu);  // NaN -> saturated
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) worst = max(worst, (uint32_t)__shfl_xor((int)worst, m, kWave));
  if (lane_id() == 0) atomicMax(max_err, worst);
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
__global__ void k_zero_u32(uint32_t* p) { *p = 0u; }

hipError_t launch_hw_error(int op, uint32_t first, uint32_t count, uint32_t* max_err, hipStream_t st) {
  hipLaunchKernelGGL(k_zero_u32, dim3(1), dim3(1), 0, st, max_err);
  const uint64_t blocks = std::min<uint64_t>(4096, ((uint64_t)count + 255) / 256);
  hipLaunchKernelGGL(k_hw_error, dim3((unsigned)blocks), dim3(256), 0, st, op, first, count, max_err);
  return hipGetLastError();
}

hipError_t launch_math_probe(const float* in, float* out_exp, float* out_log, float* out_expm1, float* out_tanh,
                             int64_t n, hipStream_t st) {
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(k_math_probe, dim3((unsigned)blocks), dim3(256), 0, st, in, out_exp, out_log, out_expm1,
                     out_tanh, n);
  return hipGetLastError();
}

hipError_t launch_penalty(const float* logits, int64_t stride, int rows, int n, const uint32_t* prev,
                          int n_prev, int64_t prev_stride, int window, float penalty, uint32_t xf, float cap,
                          float inv_scale, float* out, hipStream_t st) {
  dim3 grid((n + kMaxNT * kMaxPerThread - 1) / (kMaxNT * kMaxPerThread), rows);
  hipLaunchKernelGGL(k_penalty, grid, dim3(kMaxNT), 0, st, logits, stride, n, prev, n_prev,
                     prev_stride, window, penalty, xf, cap, inv_scale, out);
  return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, int64_t stride, int rows, int n, uint32_t xf, float cap,
                         float inv_scale, uint32_t* tokens, uint8_t* consumed, uint32_t* kept_count,
                         uint32_t* path, hipStream_t st) {
  hipLaunchKernelGGL(k_argmax, dim3(rows), dim3(kNT), 0, st, logits, stride, n, xf, cap, inv_scale, tokens,
                     consumed, kept_count, path);
  return hipGetLastError();
}


}  // namespace llz
