// coef.hip - per-chunk coefficients of the chunked closed form, for every chunk of every row.
//
// The coefficients of a chunk depend only on its decay / lr / beta / gate values, never on the
// states, so they are formed here ahead of the segment walks, with one small workgroup per
// (chunk, bh) and many workgroups per CU: the step-by-step recurrences that would otherwise sit on
// a walk's critical path overlap across chunks. Per chunk:
//   record (fp32): acoef[CH] = a_{t-1}, kcoef[CH] = kappa_{t-1}, endc = (a, kappa, b) of the chunk,
//                  wsend[SPM] = Ws[s, end], wzend[SPM] = Wz[s, end]
//   wsh (T):       Ws[s, t-1] as [CH][SPM] (optional)
// The walks prefetch these with the chunk's other inputs.
#include "mem_common.h"
#include "mem_params.h"
#include "seg_common.h"

namespace atlas {

constexpr int kCoefThreads = 128;   // two waves: sources 0..127, prefix chain in lane 127

template <typename T, int CH, bool WSH>
__global__ __launch_bounds__(kCoefThreads) void k_chunk_coef(const Geom g, const T* __restrict__ decay,
                                                               const T* __restrict__ lr, const T* __restrict__ beta,
                                                               const T* __restrict__ gate, float* __restrict__ rec,
                                                               T* __restrict__ wsh) {
  constexpr int SPM = CH + kHaloPad;
  constexpr int REC = CoefRec<CH>::SIZE;
  __shared__ ChunkScalars<CH> sc;
  const int c = blockIdx.x, bh = blockIdx.y, tid = threadIdx.x;
  const int H = g.H, e = g.e;
  const int t0 = c * g.Lc, L = min(g.T, t0 + g.Lc) - t0;
  const size_t tb = (size_t)bh * g.T, r0 = tb + t0;
  for (int t = tid; t < CH; t += kCoefThreads) {
    const bool ok = t < L;
    const size_t rt = ok ? r0 + t : r0;
    const T x_al = decay[rt], x_et = lr[rt], x_be = (g.momentum && beta ? beta : decay)[rt];
    sc.alpha[t] = ok ? to_f32(x_al) : 1.f;
    sc.eta[t] = ok ? to_f32(x_et) : 0.f;
    sc.beta[t] = ok ? (g.momentum ? to_f32(x_be) : 0.f) : 1.f;
  }
  if (g.gate_mode == GATE_TOKEN) {
    for (int s = tid; s < SPM; s += kCoefThreads) {
      const int p = t0 - H + s;
      const bool in = s < H + L;
      const T x = gate[(in && p >= 0) ? tb + p : r0];
      sc.ug[s] = in ? (p >= 0 ? to_f32(x) : 1.f) : 0.f;
    }
  } else if (g.gate_mode == GATE_LAG) {
    for (int idx = tid; idx < CH * e; idx += kCoefThreads) {
      const bool ok = idx / e < L;
      const T x = gate[ok ? r0 * e + idx : r0];
      sc.wl[idx] = ok ? to_f32(x) : 0.f;
    }
  }
  __syncthreads();
  T* w = WSH ? wsh + ((size_t)bh * g.nc + c) * CH * SPM : nullptr;
  chunk_coefficients<CH, WSH, true, T>(g, sc, L, tid, w, SPM);
  __syncthreads();
  float4* dst = reinterpret_cast<float4*>(rec + ((size_t)bh * g.nc + c) * REC);
  const float4* src = reinterpret_cast<const float4*>(&sc.acoef[0]);
  for (int i = tid; i < REC / 4; i += kCoefThreads) dst[i] = src[i];
}

template <typename T, int CH>
hipError_t launch_chunk_coef(const Geom& g, const T* decay, const T* lr, const T* beta, const T* gate, float* rec,
                             T* wsh, int kid, hipStream_t stream) {
  prof_begin(kid, stream);
  if (wsh) {
    hipLaunchKernelGGL((k_chunk_coef<T, CH, true>), dim3(g.nc, g.BH), dim3(kCoefThreads), 0, stream, g, decay, lr,
                       beta, gate, rec, wsh);
  } else {
    hipLaunchKernelGGL((k_chunk_coef<T, CH, false>), dim3(g.nc, g.BH), dim3(kCoefThreads), 0, stream, g, decay, lr,
                       beta, gate, rec, wsh);
  }
  prof_end(kid, stream);
  return hipGetLastError();
}

#define ATLAS_INST_COEF(T, CH)                                                                        \
  template hipError_t launch_chunk_coef<T, CH>(const Geom&, const T*, const T*, const T*, const T*, float*, \
                                               T*, int, hipStream_t);

ATLAS_INST_COEF(bf16, 64)
ATLAS_INST_COEF(float, 32)
ATLAS_INST_COEF(bf16, 32)
ATLAS_INST_COEF(float, 16)

}  // namespace atlas
