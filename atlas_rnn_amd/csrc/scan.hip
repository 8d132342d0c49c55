// scan.hip - scalar-gated associative scan and window sum primitives (gfx950).
//
//   scan:        out_t = g_t * out_{t-1} + x_t  over [N, T, D], gates [N, T], out_{-1} = prev (or 0)
//                (the AssocScan contract used at atlas_pytorch/rnn_memory.py:363,369,698,700,705 and
//                 atlas_pytorch/omega.py:267,315)
//   window sum:  y_t = sum_{k = max(0, t-w+1)}^{t} x_k  (rnn_memory.py:50-61, omega.py:24-33), summed
//                directly in fp32 rather than as a cumsum difference, so no cancellation with T.
// One thread owns one column d and walks T; consecutive threads read consecutive d (coalesced).
#include <hip/hip_runtime.h>

#include "../../include/atlas_mem.h"
#include "mem_common.h"

namespace atlas {

template <typename T>
__global__ __launch_bounds__(kThreads) void k_scan_fwd(int64_t Tn, int64_t D, const T* g, const T* x,
                                                         const T* prev, T* out) {
  const int64_t n = blockIdx.y;
  const int64_t d = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (d >= D) return;
  float cur = prev ? to_f32(prev[n * D + d]) : 0.f;
  const T* gp = g + n * Tn;
  const T* xp = x + n * Tn * D + d;
  T* op = out + n * Tn * D + d;
  for (int64_t t = 0; t < Tn; ++t) {
    cur = to_f32(gp[t]) * cur + to_f32(xp[t * D]);
    op[t * D] = from_f32<T>(cur);
  }
}

// lambda_t = dout_t + g_{t+1} lambda_{t+1};  dx_t = lambda_t;  dprev = g_0 lambda_0
template <typename T>
__global__ __launch_bounds__(kThreads) void k_scan_bwd_dx(int64_t Tn, int64_t D, const T* g, const T* dout,
                                                            T* dx, T* dprev) {
  const int64_t n = blockIdx.y;
  const int64_t d = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (d >= D) return;
  const T* gp = g + n * Tn;
  const T* dp = dout + n * Tn * D + d;
  T* xp = dx + n * Tn * D + d;
  float lam = 0.f, gnext = 0.f;
  for (int64_t t = Tn - 1; t >= 0; --t) {
    lam = to_f32(dp[t * D]) + gnext * lam;
    xp[t * D] = from_f32<T>(lam);
    gnext = to_f32(gp[t]);
  }
  if (dprev) dprev[n * D + d] = from_f32<T>(gnext * lam);
}

// dg_t = sum_d dx_t[d] * out_{t-1}[d]   (out_{-1} = prev or 0).  grid (T, N)
template <typename T>
__global__ __launch_bounds__(kThreads) void k_scan_bwd_dg(int64_t Tn, int64_t D, const T* out, const T* prev,
                                                            const T* dx, T* dg) {
  __shared__ float red[kWaves];
  const int64_t n = blockIdx.y, t = blockIdx.x;
  const T* lp = dx + (n * Tn + t) * D;
  const T* op = (t > 0) ? out + (n * Tn + t - 1) * D : (prev ? prev + n * D : nullptr);
  float acc = 0.f;
  if (op) {
    for (int64_t d = threadIdx.x; d < D; d += kThreads) acc += to_f32(lp[d]) * to_f32(op[d]);
  }
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
  if (lane_id() == 0) red[wave_id()] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.f;
    for (int w = 0; w < kWaves; ++w) s += red[w];
    dg[n * Tn + t] = from_f32<T>(s);
  }
}

// reverse == 0: y_t = sum_{k=max(0,t-w+1)}^{t} x_k ; reverse == 1: y_t = sum_{k=t}^{min(T-1,t+w-1)} x_k
template <typename T>
__global__ __launch_bounds__(kThreads) void k_window_sum(int64_t Tn, int64_t D, int w, int reverse, const T* x, T* y) {
  const int64_t n = blockIdx.y;
  const int64_t d = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (d >= D) return;
  const T* xp = x + n * Tn * D + d;
  T* yp = y + n * Tn * D + d;
  for (int64_t t = 0; t < Tn; ++t) {
    float acc = 0.f;
    if (!reverse) {
      const int64_t k0 = t - w + 1 > 0 ? t - w + 1 : 0;
      for (int64_t k = k0; k <= t; ++k) acc += to_f32(xp[k * D]);
    } else {
      const int64_t k1 = t + w - 1 < Tn - 1 ? t + w - 1 : Tn - 1;
      for (int64_t k = t; k <= k1; ++k) acc += to_f32(xp[k * D]);
    }
    yp[t * D] = from_f32<T>(acc);
  }
}

}  // namespace atlas

using namespace atlas;

namespace {
bool bad_dims(int64_t n, int64_t t, int64_t d) { return n < 1 || t < 1 || d < 1 || n > 65535; }
}

extern "C" {

int atlas_scan_fwd(int dtype, int64_t n, int64_t t, int64_t d, const void* gates, const void* x,
                   const void* prev, void* out, void* stream) {
  if (bad_dims(n, t, d)) return ATLAS_MEM_ERR_SHAPE;
  if (!gates || !x || !out) return ATLAS_MEM_ERR_NULL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((d + kThreads - 1) / kThreads), (unsigned)n);
  if (dtype == ATLAS_DT_BF16)
    hipLaunchKernelGGL(k_scan_fwd<bf16>, grid, dim3(kThreads), 0, s, t, d, (const bf16*)gates, (const bf16*)x,
                       (const bf16*)prev, (bf16*)out);
  else if (dtype == ATLAS_DT_F32)
    hipLaunchKernelGGL(k_scan_fwd<float>, grid, dim3(kThreads), 0, s, t, d, (const float*)gates, (const float*)x,
                       (const float*)prev, (float*)out);
  else
    return ATLAS_MEM_ERR_DTYPE;
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

int atlas_scan_bwd(int dtype, int64_t n, int64_t t, int64_t d, const void* gates, const void* out,
                   const void* prev, const void* dout, void* dx, void* dgates, void* dprev, void* stream) {
  if (bad_dims(n, t, d)) return ATLAS_MEM_ERR_SHAPE;
  if (!gates || !out || !dout || !dx || !dgates) return ATLAS_MEM_ERR_NULL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((d + kThreads - 1) / kThreads), (unsigned)n);
  const dim3 grid2((unsigned)t, (unsigned)n);
  if (t > 2147483647) return ATLAS_MEM_ERR_SHAPE;
  if (dtype == ATLAS_DT_BF16) {
    hipLaunchKernelGGL(k_scan_bwd_dx<bf16>, grid, dim3(kThreads), 0, s, t, d, (const bf16*)gates, (const bf16*)dout,
                       (bf16*)dx, (bf16*)dprev);
    hipLaunchKernelGGL(k_scan_bwd_dg<bf16>, grid2, dim3(kThreads), 0, s, t, d, (const bf16*)out, (const bf16*)prev,
                       (const bf16*)dx, (bf16*)dgates);
  } else if (dtype == ATLAS_DT_F32) {
    hipLaunchKernelGGL(k_scan_bwd_dx<float>, grid, dim3(kThreads), 0, s, t, d, (const float*)gates,
                       (const float*)dout, (float*)dx, (float*)dprev);
    hipLaunchKernelGGL(k_scan_bwd_dg<float>, grid2, dim3(kThreads), 0, s, t, d, (const float*)out,
                       (const float*)prev, (const float*)dx, (float*)dgates);
  } else {
    return ATLAS_MEM_ERR_DTYPE;
  }
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

int atlas_window_sum(int dtype, int64_t n, int64_t t, int64_t d, int window, int reverse, const void* x, void* y,
                     void* stream) {
  if (bad_dims(n, t, d) || window < 1) return ATLAS_MEM_ERR_SHAPE;
  if (!x || !y) return ATLAS_MEM_ERR_NULL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((d + kThreads - 1) / kThreads), (unsigned)n);
  if (dtype == ATLAS_DT_BF16)
    hipLaunchKernelGGL(k_window_sum<bf16>, grid, dim3(kThreads), 0, s, t, d, window, reverse, (const bf16*)x, (bf16*)y);
  else if (dtype == ATLAS_DT_F32)
    hipLaunchKernelGGL(k_window_sum<float>, grid, dim3(kThreads), 0, s, t, d, window, reverse, (const float*)x,
                       (float*)y);
  else
    return ATLAS_MEM_ERR_DTYPE;
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

}  // extern "C"
