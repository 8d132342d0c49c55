// mem_fwd.hip - forward helper kernel: the carried Omega buffer.
//
// buffer' = last e-1 of [buffer; Ghat_0 .. Ghat_{T-1}] with Ghat_p = u_p delta_p phi_p^T (per-token
// gate) or delta_p phi_p^T (otherwise), delta_p = S_ref phi_p - v_p   (rnn_memory.py:673-687).
#include "mem_common.h"
#include "mem_params.h"

namespace atlas {

// buffer' = last e-1 of [buffer; Ghat_0 .. Ghat_{T-1}], Ghat_p = gate_p * delta_p phi_p^T
// (token mode) or delta_p phi_p^T (otherwise).  rnn_memory.py:673-687.   grid (H, BH).
template <typename T, int DK, int DV>
__global__ __launch_bounds__(kThreads) void k_buffer_out(const Geom g, const FwdPtrs<T> a) {
  __shared__ float sphi[DK];
  __shared__ float sdel[DV];
  const int slot = blockIdx.x, bh = blockIdx.y, H = g.H;
  const int ext = g.T + slot;          // index into [buffer (H); tokens (T)]
  float* out = a.buf_out + ((size_t)bh * H + slot) * DV * DK;
  const int tid = threadIdx.x;
  if (ext < H) {
    for (int idx = tid; idx < DV * DK; idx += kThreads)
      out[idx] = g.has_buf ? a.buf_in[((size_t)bh * H + ext) * DV * DK + idx] : 0.f;
    return;
  }
  const int p = ext - H;
  const size_t tb = (size_t)bh * g.T;
  for (int k = tid; k < DK; k += kThreads) sphi[k] = ld_map(a.k, (tb + p) * DK + k, g.map_mode, g.map_deg);
  __syncthreads();
  const float gp = (g.gate_mode == GATE_TOKEN) ? to_f32(a.gate[tb + p]) : 1.f;
  for (int i = tid; i < DV; i += kThreads) {
    const float* sr = a.S_ref + ((size_t)bh * DV + i) * DK;
    float acc = 0.f;
    for (int k = 0; k < DK; ++k) acc += sr[k] * sphi[k];
    sdel[i] = gp * (acc - to_f32(a.v[(tb + p) * DV + i]));
  }
  __syncthreads();
  for (int idx = tid; idx < DV * DK; idx += kThreads) out[idx] = sdel[idx / DK] * sphi[idx % DK];
}

template <typename T, int DK, int DV>
hipError_t launch_buffer_out(const Geom& g, const FwdPtrs<T>& a, hipStream_t stream) {
  if (g.H == 0 || !a.buf_out) return hipSuccess;
  prof_begin(KID_BUFFER_OUT, stream);
  hipLaunchKernelGGL((k_buffer_out<T, DK, DV>), dim3(g.H, g.BH), dim3(kThreads), 0, stream, g, a);
  prof_end(KID_BUFFER_OUT, stream);
  return hipGetLastError();
}

template hipError_t launch_buffer_out<bf16, 64, 64>(const Geom&, const FwdPtrs<bf16>&, hipStream_t);
template hipError_t launch_buffer_out<float, 64, 64>(const Geom&, const FwdPtrs<float>&, hipStream_t);
template hipError_t launch_buffer_out<bf16, 32, 32>(const Geom&, const FwdPtrs<bf16>&, hipStream_t);
template hipError_t launch_buffer_out<float, 32, 32>(const Geom&, const FwdPtrs<float>&, hipStream_t);

}  // namespace atlas
