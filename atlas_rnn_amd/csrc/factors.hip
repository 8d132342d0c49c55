// factors.hip - the carried Omega buffer as rank-1 factors, for decode.
//
// Every slot of the dense buffer [bh, e-1, d_v, d_k] the forward carries is one outer product
// Ghat_p = g_p delta_p phi_p^T (rnn_memory.py:673-687: delta_p = S_ref phi_p - v_p, g_p the token gate
// under per-token gating, 1 otherwise). The factored form keeps the two vectors instead,
//   factors [bh, e-1, d_v + d_k] fp32, slot m = (g_p delta_p [d_v] | phi_p [d_k]),
// slot 0 the oldest as in the dense buffer: (d_v + d_k) / (d_v d_k) of the bytes (1/32 at d = 64).
//   k_mem_step_fac      one decode token with the window sum over factored slots: the state update
//                       of atlas_mem_step (step.hip) and the factor ring shifted by one slot
//   k_buffer_factors    the factors a prefill of T tokens leaves (the last e-1 of [factors_in; tokens])
//   k_buffer_expand     factors -> the dense buffer (RNNMemState.omega_buffer, atlas_mem_fwd's buffer_in)
// One wave per state row i, lane k its column (d_k <= 64), as in step.hip.
#include "mem_common.h"
#include "mem_params.h"
#include "../../include/atlas_mem.h"

namespace atlas {

namespace {

constexpr int kFacRows = 4;   // state rows (waves) per workgroup

__device__ __forceinline__ float fac_wave_sum(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
  return x;
}

template <typename T>
__global__ __launch_bounds__(64 * kFacRows) void k_mem_step_fac(
    int dk, int dv, int e, int momentum, int gate_mode, int map_mode, int deg, int clamp_final,
    const T* __restrict__ k, const T* __restrict__ q, const T* __restrict__ v, const T* __restrict__ lr,
    const T* __restrict__ decay, const T* __restrict__ beta, const T* __restrict__ gate,
    const float* __restrict__ S_ref, const float* S0, const float* Z0, const float* __restrict__ fac_in,
    T* __restrict__ y, float* S_T, float* Z_T, float* __restrict__ fac_out) {
  const int bh = blockIdx.x;
  const int i = blockIdx.y * kFacRows + (threadIdx.x >> 6);
  if (i >= dv) return;   // wave-uniform; no barriers below
  const int lane = threadIdx.x & 63;
  const bool on = lane < dk;
  const int kc = on ? lane : 0;
  const int FW = dv + dk;
  const float phi = ld_map(k, (size_t)bh * dk + kc, map_mode, deg);
  const float psi = ld_map(q, (size_t)bh * dk + kc, map_mode, deg);
  const size_t so = ((size_t)bh * dv + i) * dk + kc;
  const float s = S0[so];
  const float z = (momentum && Z0) ? Z0[so] : 0.f;
  const float delta = fac_wave_sum(on ? S_ref[so] * phi : 0.f) - to_f32(v[(size_t)bh * dv + i]);
  const float yi = fac_wave_sum(on ? s * psi : 0.f);
  const float al = to_f32(decay[bh]), et = to_f32(lr[bh]);
  float w0 = 1.f;
  if (gate_mode == ATLAS_GATE_TOKEN) w0 = to_f32(gate[bh]);
  else if (gate_mode == ATLAS_GATE_LAG) w0 = to_f32(gate[(size_t)bh * e]);
  float g = w0 * delta * phi;
  const float* fi = fac_in ? fac_in + (size_t)bh * (e - 1) * FW : nullptr;
  if (fi) {
    for (int j = 1; j < e; ++j) {   // lag j: slot e-1-j
      const float cj = gate_mode == ATLAS_GATE_LAG ? to_f32(gate[(size_t)bh * e + j]) : 1.f;
      const float* sl = fi + (size_t)(e - 1 - j) * FW;
      g += cj * sl[i] * sl[dv + kc];
    }
  }
  const float zn = momentum ? to_f32(beta[bh]) * z + g : g;
  float sn = al * s - et * zn;
  if (clamp_final) sn = clamp100(sn);
  if (lane == 0) y[(size_t)bh * dv + i] = from_f32<T>(yi);
  if (on) {
    S_T[so] = sn;
    if (momentum) Z_T[so] = zn;
  }
  if (e > 1) {   // the ring: slot m <- slot m + 1, the newest slot <- (g delta | phi)
    float* fo = fac_out + (size_t)bh * (e - 1) * FW;
    const float gd = (gate_mode == ATLAS_GATE_TOKEN ? w0 : 1.f) * delta;
    if (lane == 0) {
      for (int m = 0; m + 1 < e - 1; ++m) fo[(size_t)m * FW + i] = fi ? fi[(size_t)(m + 1) * FW + i] : 0.f;
      fo[(size_t)(e - 2) * FW + i] = gd;
    }
    if (i == 0 && on) {
      for (int m = 0; m + 1 < e - 1; ++m) fo[(size_t)m * FW + dv + kc] = fi ? fi[(size_t)(m + 1) * FW + dv + kc] : 0.f;
      fo[(size_t)(e - 2) * FW + dv + kc] = phi;
    }
  }
}

// grid (bh, e-1): slot m of row bh holds token p = T - (e-1) + m, or slot m + T of factors_in when p < 0
template <typename T>
__global__ __launch_bounds__(64 * kFacRows) void k_buffer_factors(
    int T_len, int dk, int dv, int e, int gate_mode, int map_mode, int deg, const T* __restrict__ k,
    const T* __restrict__ v, const T* __restrict__ gate, const float* __restrict__ S_ref,
    const float* __restrict__ fac_in, float* __restrict__ fac_out) {
  const int bh = blockIdx.x, m = blockIdx.y, H = e - 1, FW = dv + dk;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const bool on = lane < dk;
  const int kc = on ? lane : 0;
  float* fo = fac_out + ((size_t)bh * H + m) * FW;
  const int p = T_len - H + m;
  if (p < 0) {
    const float* src = fac_in ? fac_in + ((size_t)bh * H + m + T_len) * FW : nullptr;
    for (int u = threadIdx.x; u < FW; u += 64 * kFacRows) fo[u] = src ? src[u] : 0.f;
    return;
  }
  const size_t tb = (size_t)bh * T_len + p;
  const float phi = ld_map(k, tb * dk + kc, map_mode, deg);
  const float gp = gate_mode == ATLAS_GATE_TOKEN ? to_f32(gate[tb]) : 1.f;
  for (int i = w; i < dv; i += kFacRows) {   // wave-uniform loop
    const float acc = fac_wave_sum(on ? S_ref[((size_t)bh * dv + i) * dk + kc] * phi : 0.f);
    if (lane == 0) fo[i] = gp * (acc - to_f32(v[tb * dv + i]));
  }
  if (w == 0 && on) fo[dv + kc] = phi;
}

// grid (bh * (e-1), ceil(dv / kFacRows)): dense[s][i][k] = factors[s][i] * factors[s][dv + k]
__global__ __launch_bounds__(64 * kFacRows) void k_buffer_expand(int dk, int dv, const float* __restrict__ fac,
                                                                 float* __restrict__ dense) {
  const int sidx = blockIdx.x;
  const int i = blockIdx.y * kFacRows + (threadIdx.x >> 6);
  if (i >= dv) return;
  const int lane = threadIdx.x & 63;
  const float* f = fac + (size_t)sidx * (dv + dk);
  const float di = f[i];
  float* o = dense + ((size_t)sidx * dv + i) * dk;
  for (int kc = lane; kc < dk; kc += 64) o[kc] = di * f[dv + kc];
}

inline bool fac_misaligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) != 0; }

inline bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return a && b && x < y + nb && y < x + na;
}

}  // namespace

}  // namespace atlas

extern "C" {

int atlas_mem_step_factored(const atlas_mem_problem* prob, const atlas_mem_fwd_args* a, const float* factors_in,
                            float* factors_out, void* stream) {
  using namespace atlas;
  if (!prob || !a) return ATLAS_MEM_ERR_NULL;
  const int st = atlas_mem_validate(prob);
  if (st != ATLAS_MEM_OK && st != ATLAS_MEM_ERR_UNSUPPORTED) return st;   // clamp_every has no effect at T = 1
  const atlas_mem_problem& p = *prob;
  if (p.seq_len != 1 || p.d_k > 64) return ATLAS_MEM_ERR_SHAPE;
  if (!a->k || !a->q || !a->v || !a->lr || !a->decay || !a->S_ref || !a->S0 || !a->y || !a->S_T)
    return ATLAS_MEM_ERR_NULL;
  if (p.momentum && (!a->beta || !a->Z_T)) return ATLAS_MEM_ERR_NULL;
  if (!p.momentum && (a->beta || a->Z_T)) return ATLAS_MEM_ERR_ARG;
  if ((p.gate_mode != ATLAS_GATE_NONE) != (a->gate != nullptr)) return ATLAS_MEM_ERR_ARG;
  if (a->buffer_in || a->buffer_out) return ATLAS_MEM_ERR_ARG;   // the dense buffer is not used here
  if (p.has_buffer && !factors_in) return ATLAS_MEM_ERR_NULL;
  if (p.window > 1 && !factors_out) return ATLAS_MEM_ERR_NULL;
  const void* ptrs[] = {a->k, a->q, a->v, a->lr, a->decay, a->beta, a->gate, a->y, a->S_ref, a->S0, a->Z0,
                        a->S_T, a->Z_T, factors_in, factors_out};
  for (const void* q : ptrs) if (fac_misaligned(q)) return ATLAS_MEM_ERR_ALIGN;
  const int e = p.window;
  const size_t fbytes = (size_t)p.bh * (e > 1 ? e - 1 : 0) * (p.d_v + p.d_k) * sizeof(float);
  if (p.has_buffer && overlaps(factors_in, fbytes, factors_out, fbytes)) return ATLAS_MEM_ERR_ARG;
  const int deg = p.map_mode == ATLAS_MAP_ELEMENTWISE ? p.map_degree : 1;
  const float* fin = p.has_buffer ? factors_in : nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(p.bh, (p.d_v + kFacRows - 1) / kFacRows), block(64 * kFacRows);
  if (p.dtype == ATLAS_DT_BF16) {
    hipLaunchKernelGGL(k_mem_step_fac<bf16>, grid, block, 0, s, p.d_k, p.d_v, e, p.momentum, p.gate_mode, p.map_mode,
                       deg, p.clamp_final, (const bf16*)a->k, (const bf16*)a->q, (const bf16*)a->v,
                       (const bf16*)a->lr, (const bf16*)a->decay, (const bf16*)a->beta, (const bf16*)a->gate,
                       a->S_ref, a->S0, a->Z0, fin, (bf16*)a->y, a->S_T, a->Z_T, factors_out);
  } else {
    hipLaunchKernelGGL(k_mem_step_fac<float>, grid, block, 0, s, p.d_k, p.d_v, e, p.momentum, p.gate_mode, p.map_mode,
                       deg, p.clamp_final, (const float*)a->k, (const float*)a->q, (const float*)a->v,
                       (const float*)a->lr, (const float*)a->decay, (const float*)a->beta, (const float*)a->gate,
                       a->S_ref, a->S0, a->Z0, fin, (float*)a->y, a->S_T, a->Z_T, factors_out);
  }
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

int atlas_buffer_factors(const atlas_mem_problem* prob, const void* k, const void* v, const void* gate,
                         const float* S_ref, const float* factors_in, float* factors_out, void* stream) {
  using namespace atlas;
  if (!prob) return ATLAS_MEM_ERR_NULL;
  const int st = atlas_mem_validate(prob);
  if (st != ATLAS_MEM_OK && st != ATLAS_MEM_ERR_UNSUPPORTED) return st;
  const atlas_mem_problem& p = *prob;
  if (p.window < 2 || p.d_k > 64) return ATLAS_MEM_ERR_SHAPE;
  if (!k || !v || !S_ref || !factors_out) return ATLAS_MEM_ERR_NULL;
  if ((p.gate_mode != ATLAS_GATE_NONE) != (gate != nullptr)) return ATLAS_MEM_ERR_ARG;
  if (p.has_buffer && !factors_in) return ATLAS_MEM_ERR_NULL;
  for (const void* q : {k, v, gate, (const void*)S_ref, (const void*)factors_in, (const void*)factors_out})
    if (fac_misaligned(q)) return ATLAS_MEM_ERR_ALIGN;
  const size_t fbytes = (size_t)p.bh * (p.window - 1) * (p.d_v + p.d_k) * sizeof(float);
  if (p.has_buffer && overlaps(factors_in, fbytes, factors_out, fbytes)) return ATLAS_MEM_ERR_ARG;
  const int deg = p.map_mode == ATLAS_MAP_ELEMENTWISE ? p.map_degree : 1;
  const float* fin = p.has_buffer ? factors_in : nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(p.bh, p.window - 1), block(64 * kFacRows);
  if (p.dtype == ATLAS_DT_BF16)
    hipLaunchKernelGGL(k_buffer_factors<bf16>, grid, block, 0, s, p.seq_len, p.d_k, p.d_v, p.window, p.gate_mode,
                       p.map_mode, deg, (const bf16*)k, (const bf16*)v, (const bf16*)gate, S_ref, fin, factors_out);
  else
    hipLaunchKernelGGL(k_buffer_factors<float>, grid, block, 0, s, p.seq_len, p.d_k, p.d_v, p.window, p.gate_mode,
                       p.map_mode, deg, (const float*)k, (const float*)v, (const float*)gate, S_ref, fin,
                       factors_out);
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

int atlas_buffer_expand(int bh, int slots, int d_v, int d_k, const float* factors, float* dense, void* stream) {
  using namespace atlas;
  if (bh < 1 || slots < 0 || d_v < 1 || d_k < 1 || d_v > 65536 || d_k > 65536 || (int64_t)bh * slots > 2147483647)
    return ATLAS_MEM_ERR_SHAPE;
  if (slots == 0) return ATLAS_MEM_OK;
  if (!factors || !dense) return ATLAS_MEM_ERR_NULL;
  if (fac_misaligned(factors) || fac_misaligned(dense)) return ATLAS_MEM_ERR_ALIGN;
  const dim3 grid(bh * slots, (d_v + kFacRows - 1) / kFacRows), block(64 * kFacRows);
  hipLaunchKernelGGL(k_buffer_expand, grid, block, 0, static_cast<hipStream_t>(stream), d_k, d_v, factors, dense);
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

}  // extern "C"
