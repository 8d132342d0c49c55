// seg_common.h - pieces shared by the segment-parallel kernels.
#pragma once

#include "mem_common.h"
#include "mem_params.h"

namespace atlas {

constexpr int kSegThreads = 512;   // 8 waves per workgroup
constexpr int kSegWaves = kSegThreads / kWave;

struct SegGeom {
  int G;              // chunks per segment
  int nseg;           // segments per head-batch row
  int agg_stride;     // floats per segment aggregate: U, V (2 D^2) + a, kappa, b (padded to 16)
};

// Backward-pass buffers beyond the user-visible arguments.
struct BwdSegPtrs {
  const float* seg_states;   // forward segment-start states [BH][nseg][2][D][D]
  const float* final_raw;    // forward raw S_{T-1} [BH][D][D]
  float* adj_agg;            // [BH][nseg][agg_stride]: L, K, a, kappa, b
  float* rw;                 // [BH][nseg][Gb][2][D][D] raw chunk-start states of the re-walk
  float* dsref_part;         // [BH][nseg][D][D]
  float* tail_part;          // [BH][nseg][H][2D]  (dv | dphi) partial of a segment's last H tokens
  float* halo_part;          // [BH][nseg][H][2D]  partial from the segment's first chunk for the previous segment
  float* dw;                 // [BH][T][e] per (target, lag) gradients (token gates)
};

// Eight consecutive elements: one 16-byte (bf16) or two 16-byte (fp32) vector accesses.
template <typename T>
struct Vec8 {
  T v[8];
  static __device__ __forceinline__ Vec8 zero() {
    Vec8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r.v[e] = static_cast<T>(0.f);
    return r;
  }
  __device__ __forceinline__ Vec8 mapped(int deg) const {
    Vec8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r.v[e] = static_cast<T>(poly_map(to_f32(v[e]), deg));
    return r;
  }
  __device__ __forceinline__ void store(T* p) const {
    if constexpr (sizeof(T) == 2) {
      *reinterpret_cast<uint4*>(p) = *reinterpret_cast<const uint4*>(v);
    } else {
      reinterpret_cast<uint4*>(p)[0] = reinterpret_cast<const uint4*>(v)[0];
      reinterpret_cast<uint4*>(p)[1] = reinterpret_cast<const uint4*>(v)[1];
    }
  }
};

template <typename T>
__device__ __forceinline__ Vec8<T> vec8_load(const T* p) {
  Vec8<T> r;
  if constexpr (sizeof(T) == 2) {
    *reinterpret_cast<uint4*>(r.v) = *reinterpret_cast<const uint4*>(p);
  } else {
    reinterpret_cast<uint4*>(r.v)[0] = reinterpret_cast<const uint4*>(p)[0];
    reinterpret_cast<uint4*>(r.v)[1] = reinterpret_cast<const uint4*>(p)[1];
  }
  return r;
}

// Per-chunk scalars and coefficients in LDS.
template <int CH>
struct ChunkScalars {
  static constexpr int SPM = CH + kHaloPad;
  float alpha[CH], eta[CH], beta[CH];   // padded targets: alpha = beta = 1, eta = 0
  float ug[SPM];                        // token-mode gate of each source
  float wl[CH * kMaxWindow];            // lag-mode weights [tau][j]
  float wsend[SPM], wzend[SPM];         // Ws[s, end], Wz[s, end]
  float acoef[CH], kcoef[CH];           // a_{tau-1}, kappa_{tau-1}
  float endc[4];                        // a_end, kappa_end, b_end
};

// Coefficient recurrences of a chunk, run by 128 lanes (ci = 0..127):
//   source s (ci < SP):  Wz[s,t] = beta_t Wz[s,t-1] + w(s,t),  Ws[s,t] = alpha_t Ws[s,t-1] + eta_t Wz[s,t]
//                        (w(s,t) = window weight of source s at target t), writing Ws[s, t-1] to
//                        wsh[t * ldw + s] when wsh != nullptr and the end values to wsend / wzend;
//   ci == 127:           b_t = beta_t b_{t-1}, a_t = alpha_t a_{t-1}, kappa_t = alpha_t kappa_{t-1} + eta_t b_t.
template <int CH, bool WSH>
__device__ __forceinline__ void chunk_coefficients(const Geom& g, ChunkScalars<CH>& sc, int L, int ci,
                                                   float* __restrict__ wsh, int ldw) {
  const float* __restrict__ al = sc.alpha;
  const float* __restrict__ et = sc.eta;
  const float* __restrict__ be = sc.beta;
  const float* __restrict__ wl = sc.wl;
  const int H = g.H, e = g.e;
  if (ci < g.SP) {
    const int s = ci;
    const float us = g.gate_mode == GATE_TOKEN ? sc.ug[s] : 1.f;
    float ws = 0.f, wz = 0.f;
#pragma unroll 8
    for (int t = 0; t < CH; ++t) {
      if constexpr (WSH) wsh[t * ldw + s] = ws;
      const int j = t + H - s;
      float w = 0.f;
      if (j >= 0 && j < e && t < L) w = (g.gate_mode == GATE_LAG) ? wl[t * e + j] : us;
      wz = be[t] * wz + w;
      ws = al[t] * ws + et[t] * wz;
    }
    sc.wsend[s] = ws;
    sc.wzend[s] = wz;
  } else if (ci == 127) {
    float ac = 1.f, kc = 0.f, bc = 1.f;
    for (int t = 0; t < CH; ++t) {
      sc.acoef[t] = ac;
      sc.kcoef[t] = kc;
      bc = be[t] * bc;
      ac = al[t] * ac;
      kc = al[t] * kc + et[t] * bc;
    }
    sc.endc[0] = ac; sc.endc[1] = kc; sc.endc[2] = bc;
  }
}

}  // namespace atlas
