// step.hip - one token of the memory recurrence (decode / streaming): atlas_mem_step.
//
// The same recurrence as atlas_mem_fwd at T = 1 (rnn_memory.py:659-728; one iteration of the
// per-token loop), for generation, where every call carries one token and the state:
//   y = S0 psi,  delta = S_ref phi - v,  P = delta phi^T,
//   g = w0 P + sum_{j=1..e-1} c_j buffer[e-1-j],   (lag gates: w0 = U[0], c_j = U[j]; token gate:
//                                                   w0 = u, c_j = 1; none: 1)
//   Z_T = beta Z0 + g (momentum) ,  S_T = alpha S0 - eta Z_T (or - eta g),  clamped to +-100,
//   buffer_out = [buffer[1 .. e-2], (token gate: u) P].
// Every state element is independent of the others apart from the two row sums (delta_i and y_i),
// so one wave owns one state row i, lane k its column: the row sums are wave reductions and every
// state access is one coalesced 4-byte load or store per lane. The kernel reads S_ref, S0, Z0 and
// the buffer once and writes S_T, Z_T and the buffer once: HBM-bound at
// BH d_v d_k 4 B (3 + momentum 2 + 2 (e-1)) per step. Outputs may alias their inputs (S_T = S0,
// Z_T = Z0, buffer_out = buffer_in): each element is read before it is written, by the same lane.
#include "mem_common.h"
#include "mem_params.h"
#include "../../include/atlas_mem.h"

namespace atlas {

namespace {

constexpr int kStepRows = 4;   // state rows per workgroup, one wave each

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
  return x;
}

template <typename T>
__global__ __launch_bounds__(64 * kStepRows) void k_mem_step(
    int dk, int dv, int e, int momentum, int gate_mode, int map_mode, int deg, int clamp_final,
    const T* __restrict__ k, const T* __restrict__ q, const T* __restrict__ v, const T* __restrict__ lr,
    const T* __restrict__ decay, const T* __restrict__ beta, const T* __restrict__ gate,
    const float* __restrict__ S_ref, const float* S0, const float* Z0, const float* buf_in, T* __restrict__ y,
    float* S_T, float* Z_T, float* buf_out) {
  const int bh = blockIdx.x;
  const int i = blockIdx.y * kStepRows + (threadIdx.x >> 6);
  if (i >= dv) return;   // wave-uniform; no barriers below
  const int lane = threadIdx.x & 63;
  const bool on = lane < dk;
  const int kc = on ? lane : 0;
  const float phi = ld_map(k, (size_t)bh * dk + kc, map_mode, deg);
  const float psi = ld_map(q, (size_t)bh * dk + kc, map_mode, deg);
  const size_t so = ((size_t)bh * dv + i) * dk + kc;
  const float s = S0[so];
  const float z = (momentum && Z0) ? Z0[so] : 0.f;
  const float delta = wave_sum(on ? S_ref[so] * phi : 0.f) - to_f32(v[(size_t)bh * dv + i]);
  const float yi = wave_sum(on ? s * psi : 0.f);
  const float P = delta * phi;
  const float al = to_f32(decay[bh]), et = to_f32(lr[bh]);
  float w0 = 1.f;
  if (gate_mode == ATLAS_GATE_TOKEN) w0 = to_f32(gate[bh]);
  else if (gate_mode == ATLAS_GATE_LAG) w0 = to_f32(gate[(size_t)bh * e]);
  float g = w0 * P;
  const size_t plane = (size_t)dv * dk;
  const size_t bb = (size_t)bh * (e - 1) * plane + (size_t)i * dk + kc;   // buffer slot 0 of this element
  if (buf_in) {
    for (int j = 1; j < e; ++j) {
      const float cj = gate_mode == ATLAS_GATE_LAG ? to_f32(gate[(size_t)bh * e + j]) : 1.f;
      g += cj * buf_in[bb + (size_t)(e - 1 - j) * plane];
    }
  }
  const float zn = momentum ? to_f32(beta[bh]) * z + g : g;
  float sn = al * s - et * zn;
  if (clamp_final) sn = clamp100(sn);
  if (lane == 0) y[(size_t)bh * dv + i] = from_f32<T>(yi);
  if (!on) return;
  S_T[so] = sn;
  if (momentum) Z_T[so] = zn;
  if (e > 1) {
    // slot m takes slot m + 1 (read before slot m + 1 is written, so in place is safe)
    for (int m = 0; m + 1 < e - 1; ++m) buf_out[bb + (size_t)m * plane] = buf_in ? buf_in[bb + (size_t)(m + 1) * plane] : 0.f;
    buf_out[bb + (size_t)(e - 2) * plane] = gate_mode == ATLAS_GATE_TOKEN ? w0 * P : P;
  }
}

inline bool misaligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) != 0; }

}  // namespace

}  // namespace atlas

extern "C" int atlas_mem_step(const atlas_mem_problem* prob, const atlas_mem_fwd_args* a, void* stream) {
  using namespace atlas;
  if (!prob || !a) return ATLAS_MEM_ERR_NULL;
  const int st = atlas_mem_validate(prob);
  if (st != ATLAS_MEM_OK && st != ATLAS_MEM_ERR_UNSUPPORTED) return st;   // clamp_every has no effect at T = 1
  const atlas_mem_problem& p = *prob;
  if (p.seq_len != 1) return ATLAS_MEM_ERR_SHAPE;
  if (!a->k || !a->q || !a->v || !a->lr || !a->decay || !a->S_ref || !a->S0 || !a->y || !a->S_T)
    return ATLAS_MEM_ERR_NULL;
  if (p.momentum && (!a->beta || !a->Z_T)) return ATLAS_MEM_ERR_NULL;
  if (!p.momentum && (a->beta || a->Z_T)) return ATLAS_MEM_ERR_ARG;
  if ((p.gate_mode != ATLAS_GATE_NONE) != (a->gate != nullptr)) return ATLAS_MEM_ERR_ARG;
  if (p.has_buffer && !a->buffer_in) return ATLAS_MEM_ERR_NULL;
  if (p.window > 1 && !a->buffer_out) return ATLAS_MEM_ERR_NULL;
  const void* ptrs[] = {a->k, a->q, a->v, a->lr, a->decay, a->beta, a->gate, a->y, a->S_ref, a->S0, a->Z0,
                        a->buffer_in, a->S_T, a->Z_T, a->buffer_out};
  for (const void* q : ptrs) if (misaligned16(q)) return ATLAS_MEM_ERR_ALIGN;
  const int e = p.window;
  const int deg = p.map_mode == ATLAS_MAP_ELEMENTWISE ? p.map_degree : 1;
  const float* buf_in = p.has_buffer ? a->buffer_in : nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(p.bh, (p.d_v + kStepRows - 1) / kStepRows), block(64 * kStepRows);
  if (p.dtype == ATLAS_DT_BF16) {
    hipLaunchKernelGGL(k_mem_step<bf16>, grid, block, 0, s, p.d_k, p.d_v, e, p.momentum, p.gate_mode, p.map_mode, deg,
                       p.clamp_final, (const bf16*)a->k, (const bf16*)a->q, (const bf16*)a->v, (const bf16*)a->lr,
                       (const bf16*)a->decay, (const bf16*)a->beta, (const bf16*)a->gate, a->S_ref, a->S0, a->Z0,
                       buf_in, (bf16*)a->y, a->S_T, a->Z_T, a->buffer_out);
  } else {
    hipLaunchKernelGGL(k_mem_step<float>, grid, block, 0, s, p.d_k, p.d_v, e, p.momentum, p.gate_mode, p.map_mode, deg,
                       p.clamp_final, (const float*)a->k, (const float*)a->q, (const float*)a->v, (const float*)a->lr,
                       (const float*)a->decay, (const float*)a->beta, (const float*)a->gate, a->S_ref, a->S0, a->Z0,
                       buf_in, (float*)a->y, a->S_T, a->Z_T, a->buffer_out);
  }
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}
