// buffer_out.h - the carried Omega buffer of the forward pass:
//   buffer' = last e-1 of [buffer; Ghat_0 .. Ghat_{T-1}],  Ghat_p = u_p delta_p phi_p^T (per-token
//   gate) or delta_p phi_p^T (otherwise),  delta_p = S_ref phi_p - v_p   (rnn_memory.py:673-687).
// It depends on the inputs only; the forward runs it as extra workgroups of its segment-scan launch
// (seg_fwd.hip), one workgroup of kThreads threads per (slot, bh).
#pragma once

#include "mem_common.h"
#include "mem_params.h"

namespace atlas {

template <typename T, int DK, int DV>
__device__ __forceinline__ void buffer_out_slot(const Geom& g, const FwdPtrs<T>& a, int slot, int bh) {
  __shared__ float sphi[DK];
  __shared__ float sdel[DV];
  const int H = g.H;
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
  // delta = S_ref phi - v: NP threads per row i, each over DK / NP columns in 16-byte loads, summed
  // across the NP lanes. Every global load (S_ref, v, the gate, phi) is issued before the barrier
  // that publishes phi, so the slot waits for one memory round trip.
  constexpr int NP = kThreads / DV, KP = DK / NP;
  static_assert(kThreads % DV == 0 && DK % (4 * NP) == 0 && (NP & (NP - 1)) == 0, "row split");
  const int i = tid / NP, kp = tid % NP;
  const float4* sr = reinterpret_cast<const float4*>(a.S_ref + ((size_t)bh * DV + i) * DK + kp * KP);
  float4 x[KP / 4];
#pragma unroll
  for (int u = 0; u < KP / 4; ++u) x[u] = sr[u];
  const float vp = to_f32(a.v[(tb + p) * DV + i]);
  const float gp = (g.gate_mode == GATE_TOKEN) ? to_f32(a.gate[tb + p]) : 1.f;
  for (int k = tid; k < DK; k += kThreads) sphi[k] = ld_map(a.k, (tb + p) * DK + k, g.map_mode, g.map_deg);
  __syncthreads();
  {
    float acc = 0.f;
#pragma unroll
    for (int u = 0; u < KP / 4; ++u) {
      const int k = kp * KP + 4 * u;
      acc += x[u].x * sphi[k] + x[u].y * sphi[k + 1] + x[u].z * sphi[k + 2] + x[u].w * sphi[k + 3];
    }
#pragma unroll
    for (int o = NP / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    if (kp == 0) sdel[i] = gp * (acc - vp);
  }
  __syncthreads();
  for (int idx = tid; idx < DV * DK; idx += kThreads) out[idx] = sdel[idx / DK] * sphi[idx % DK];
}

}  // namespace atlas
