// affine.hip - right-affine scan H_t = H_{t-1} A_t + B_t (atlas_pytorch/affine_scan.py:36-158).
//
// A: [N][T][D][D], B: [N][T][R][D], prev = H_0: [N][R][D] (optional, zero when absent); out holds
// H_1 .. H_T as [N][T][R][D]. fp32, one 256-thread workgroup per n, D, R <= 64. Each step stages
// A_t in LDS (padded rows, conflict-free column reads) and every thread forms R*D/256 outputs as
// fp32 dot products. The backward walks the steps in reverse with the adjoint G_t of H_t:
//   dB_t = G_t,   dA_t = H_{t-1}^T G_t,   G_{t-1} = dout_{t-1} + G_t A_t^T,   dprev = G_0.
#include <hip/hip_runtime.h>

#include "../../include/atlas_mem.h"

namespace atlas {

constexpr int kAffThreads = 256;
constexpr int kAffMax = 64;

__global__ __launch_bounds__(kAffThreads) void k_affine_scan_fwd(int T, int R, int D, const float* __restrict__ A,
                                                                   const float* __restrict__ B,
                                                                   const float* __restrict__ prev,
                                                                   float* __restrict__ out) {
  __shared__ float sh[kAffMax][kAffMax + 1];   // H_{t-1}
  __shared__ float sa[kAffMax][kAffMax + 1];   // A_t
  const int n = blockIdx.x, tid = threadIdx.x;
  const size_t aN = (size_t)n * T * D * D, bN = (size_t)n * T * R * D;
  for (int idx = tid; idx < R * D; idx += kAffThreads)
    sh[idx / D][idx % D] = prev ? prev[(size_t)n * R * D + idx] : 0.f;
  for (int t = 0; t < T; ++t) {
    const float* At = A + aN + (size_t)t * D * D;
    const float* Bt = B + bN + (size_t)t * R * D;
    for (int idx = tid; idx < D * D; idx += kAffThreads) sa[idx / D][idx % D] = At[idx];
    __syncthreads();
    float acc[kAffMax * kAffMax / kAffThreads];
#pragma unroll
    for (int j = 0; j < kAffMax * kAffMax / kAffThreads; ++j) {
      const int idx = tid + j * kAffThreads;
      acc[j] = 0.f;
      if (idx < R * D) {
        const int r = idx / D, e = idx % D;
        float s = Bt[idx];
        for (int d = 0; d < D; ++d) s += sh[r][d] * sa[d][e];
        acc[j] = s;
      }
    }
    __syncthreads();
    float* Ht = out + bN + (size_t)t * R * D;
#pragma unroll
    for (int j = 0; j < kAffMax * kAffMax / kAffThreads; ++j) {
      const int idx = tid + j * kAffThreads;
      if (idx < R * D) {
        sh[idx / D][idx % D] = acc[j];
        Ht[idx] = acc[j];
      }
    }
  }
}

__global__ __launch_bounds__(kAffThreads) void k_affine_scan_bwd(int T, int R, int D, const float* __restrict__ A,
                                                                   const float* __restrict__ H,
                                                                   const float* __restrict__ prev,
                                                                   const float* __restrict__ dout,
                                                                   float* __restrict__ dA, float* __restrict__ dB,
                                                                   float* __restrict__ dprev) {
  __shared__ float sg[kAffMax][kAffMax + 1];   // G_t
  __shared__ float sa[kAffMax][kAffMax + 1];   // A_t
  __shared__ float sp[kAffMax][kAffMax + 1];   // H_{t-1}
  const int n = blockIdx.x, tid = threadIdx.x;
  const size_t aN = (size_t)n * T * D * D, bN = (size_t)n * T * R * D;
  constexpr int PER = kAffMax * kAffMax / kAffThreads;
  for (int idx = tid; idx < R * D; idx += kAffThreads) sg[idx / D][idx % D] = dout[bN + (size_t)(T - 1) * R * D + idx];
  for (int t = T - 1; t >= 0; --t) {
    const float* At = A + aN + (size_t)t * D * D;
    const float* Hp = t > 0 ? H + bN + (size_t)(t - 1) * R * D : (prev ? prev + (size_t)n * R * D : nullptr);
    for (int idx = tid; idx < D * D; idx += kAffThreads) sa[idx / D][idx % D] = At[idx];
    for (int idx = tid; idx < R * D; idx += kAffThreads) sp[idx / D][idx % D] = Hp ? Hp[idx] : 0.f;
    __syncthreads();
    // dB_t = G_t; dA_t[d][e] = sum_r H_{t-1}[r][d] G_t[r][e]
    float* dBt = dB + bN + (size_t)t * R * D;
    for (int idx = tid; idx < R * D; idx += kAffThreads) dBt[idx] = sg[idx / D][idx % D];
    float* dAt = dA + aN + (size_t)t * D * D;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int idx = tid + j * kAffThreads;
      if (idx < D * D) {
        const int d = idx / D, e = idx % D;
        float s = 0.f;
        for (int r = 0; r < R; ++r) s += sp[r][d] * sg[r][e];
        dAt[idx] = s;
      }
    }
    // G_{t-1}[r][d] = dout_{t-1}[r][d] + sum_e G_t[r][e] A_t[d][e]
    float acc[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int idx = tid + j * kAffThreads;
      acc[j] = 0.f;
      if (idx < R * D) {
        const int r = idx / D, d = idx % D;
        float s = t > 0 ? dout[bN + (size_t)(t - 1) * R * D + idx] : 0.f;
        for (int e = 0; e < D; ++e) s += sg[r][e] * sa[d][e];
        acc[j] = s;
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int idx = tid + j * kAffThreads;
      if (idx < R * D) sg[idx / D][idx % D] = acc[j];
    }
  }
  __syncthreads();
  if (dprev)
    for (int idx = tid; idx < R * D; idx += kAffThreads) dprev[(size_t)n * R * D + idx] = sg[idx / D][idx % D];
}

}  // namespace atlas

using namespace atlas;

namespace {
int affine_check(int n, int t, int r, int d) {
  if (n < 1 || t < 1 || r < 1 || d < 1 || r > kAffMax || d > kAffMax) return ATLAS_MEM_ERR_SHAPE;
  return ATLAS_MEM_OK;
}
}  // namespace

extern "C" {

int atlas_affine_scan_fwd(int n, int t, int r, int d, const float* A, const float* B, const float* prev, float* out,
                          void* stream) {
  const int st = affine_check(n, t, r, d);
  if (st != ATLAS_MEM_OK) return st;
  if (!A || !B || !out) return ATLAS_MEM_ERR_NULL;
  hipLaunchKernelGGL(k_affine_scan_fwd, dim3(n), dim3(kAffThreads), 0, static_cast<hipStream_t>(stream), t, r, d, A, B,
                     prev, out);
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

int atlas_affine_scan_bwd(int n, int t, int r, int d, const float* A, const float* H, const float* prev,
                          const float* dout, float* dA, float* dB, float* dprev, void* stream) {
  const int st = affine_check(n, t, r, d);
  if (st != ATLAS_MEM_OK) return st;
  if (!A || !H || !dout || !dA || !dB) return ATLAS_MEM_ERR_NULL;
  hipLaunchKernelGGL(k_affine_scan_bwd, dim3(n), dim3(kAffThreads), 0, static_cast<hipStream_t>(stream), t, r, d, A, H,
                     prev, dout, dA, dB, dprev);
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

}  // extern "C"
