// seg_bwd.hip - segment-parallel backward pass of the chunked memory recurrence (gfx950).
//
// Same segments as the forward pass (one workgroup per (segment, bh), 8 waves), chunks of Lb tokens
// (Lb <= 32 for bf16, <= 16 for fp32 so that every operand of a chunk fits in LDS):
//   k_bwd_seg_agg : reverse walk of the segment's chunks from a zero adjoint -> adjoint aggregate
//                   (the transposed 2x2 transition and the local chunk-start adjoint L, K):
//                     dS_in = a dS_end + sum_t a_{t-1} dy_t psi_t^T
//                     dZ_in = b dZ_end - kappa dS_end - sum_t kappa_{t-1} dy_t psi_t^T
//   k_bwd_seg     : folds the aggregates of the following segments into the adjoint at the segment
//                   end, re-walks the forward recurrence of the segment from its saved start state
//                   (raw chunk-start states to a short-lived scratch), then walks the chunks in
//                   reverse forming every gradient of each chunk in closed form (see k_bwd_seg's
//                   phase comments) while carrying (dS, dZ) and the halo gradients of the previous
//                   chunk's last e-1 tokens.
//   k_bwd_seg_fixup : merges the partial (dv, dphi) of tokens whose window crosses a segment boundary,
//                   adds the d buffer_out terms, reduces token-gate gradients and dS_ref partials.
#include "mem_common.h"
#include "mem_params.h"
#include "seg_common.h"
#include "seg_fwd.h"

namespace atlas {


// ---------------------------------------------------------------------------------------------
// adjoint aggregates
// ---------------------------------------------------------------------------------------------
template <typename T, int CH, int D>
struct BwdAggSmem {
  T psiT[D][CH + 8];
  T dyT[D][CH + 8];
  ChunkScalars<CH> sc;
};

template <typename T, int CH, int D>
__global__ __launch_bounds__(kSegThreads) void k_bwd_seg_agg(const Geom g, const BwdPtrs<T> a, const SegGeom sg,
                                                               const BwdSegPtrs p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  typedef BwdAggSmem<T, CH, D> Sm;
  Sm& sm = *reinterpret_cast<Sm*>(smem_raw);
  constexpr int NTD = D / 16;
  constexpr int NT2 = (NTD * NTD + kSegWaves - 1) / kSegWaves;   // state tiles per wave
  typedef MM<T> M;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int seg = blockIdx.x, bh = blockIdx.y;
  const size_t tb = (size_t)bh * g.T;
  const int c_begin = seg * sg.G, c_end = min(g.nc, c_begin + sg.G);
  float lam[NT2][4], mu[NT2][4];
#pragma unroll
  for (int j = 0; j < NT2; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) { lam[j][r] = 0.f; mu[j][r] = 0.f; }
  float pa = 1.f, pk = 0.f, pb = 1.f;
  for (int c = c_end - 1; c >= c_begin; --c) {
    const int t0 = c * g.Lc, t1 = min(g.T, t0 + g.Lc), L = t1 - t0;
    __syncthreads();
    for (int idx = tid; idx < CH * D; idx += kSegThreads) {
      const int t = idx / D, k = idx % D;
      float ps = 0.f, dv = 0.f;
      if (t < L) {
        ps = ld_map(a.q, (tb + t0 + t) * D + k, g.map_mode, g.map_deg);
        dv = a.dy ? to_f32(a.dy[(tb + t0 + t) * D + k]) : 0.f;
      }
      sm.psiT[k][t] = from_f32<T>(ps);
      sm.dyT[k][t] = from_f32<T>(dv);
    }
    if (tid < CH) {
      const bool in = tid < L;
      sm.sc.alpha[tid] = in ? to_f32(a.decay[tb + t0 + tid]) : 1.f;
      sm.sc.eta[tid] = in ? to_f32(a.lr[tb + t0 + tid]) : 0.f;
      sm.sc.beta[tid] = in ? (g.momentum ? to_f32(a.beta[tb + t0 + tid]) : 0.f) : 1.f;
    }
    __syncthreads();
    if (tid == 0) {
      float ac = 1.f, kc = 0.f, bc = 1.f;
      for (int t = 0; t < CH; ++t) {
        sm.sc.acoef[t] = ac; sm.sc.kcoef[t] = kc;
        bc = sm.sc.beta[t] * bc; ac = sm.sc.alpha[t] * ac; kc = sm.sc.alpha[t] * kc + sm.sc.eta[t] * bc;
      }
      sm.sc.endc[0] = ac; sm.sc.endc[1] = kc; sm.sc.endc[2] = bc;
    }
    __syncthreads();
    const float ae = sm.sc.endc[0], ke = sm.sc.endc[1], be = sm.sc.endc[2];
#pragma unroll
    for (int j = 0; j < NT2; ++j) {
      const int tile = wave + kSegWaves * j;
      if (tile >= NTD * NTD) continue;
      const int m0 = (tile / NTD) * 16, n0 = (tile % NTD) * 16;
      f32x4 aa = zero4(), ak = zero4();
      for (int k0 = 0; k0 < CH; k0 += M::KS) {
        const typename M::frag fb = frag_ld_row<T>(&sm.psiT[0][0], CH + 8, n0, k0);
        aa = M::mma(frag_ld_kscaled<T>(&sm.dyT[0][0], CH + 8, 1, m0, k0, sm.sc.acoef), fb, aa);
        ak = M::mma(frag_ld_kscaled<T>(&sm.dyT[0][0], CH + 8, 1, m0, k0, sm.sc.kcoef), fb, ak);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float l_out = lam[j][r];
        lam[j][r] = ae * l_out + aa[r];
        mu[j][r] = g.momentum ? (be * mu[j][r] - ke * l_out - ak[r]) : 0.f;
      }
    }
    const float na = pa * ae, nk = pa * ke + pk * be;
    pb = pb * be; pa = na; pk = nk;
  }
  float* ag = p.adj_agg + ((size_t)bh * sg.nseg + seg) * sg.agg_stride;
#pragma unroll
  for (int j = 0; j < NT2; ++j) {
    const int tile = wave + kSegWaves * j;
    if (tile >= NTD * NTD) continue;
    const int m0 = (tile / NTD) * 16, n0 = (tile % NTD) * 16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = m0 + 4 * (lane >> 4) + r, k = n0 + (lane & 15);
      ag[(size_t)i * D + k] = lam[j][r];
      ag[(size_t)D * D + (size_t)i * D + k] = mu[j][r];
    }
  }
  if (tid == 0) { ag[2 * D * D] = pa; ag[2 * D * D + 1] = pk; ag[2 * D * D + 2] = pb; }
}

// ---------------------------------------------------------------------------------------------
// main reverse walk
// ---------------------------------------------------------------------------------------------
template <typename T, int CH, int D>
struct BwdSegSmem {
  static constexpr int SPM = CH + kHaloPad;
  static constexpr bool kStatesInLds = sizeof(T) == 2;   // fp32 reads S_in / Z_in from the re-walk scratch
  T sref[D][D + 8];
  T dSe[D][D + 8];
  T dZe[D][D + 8];
  T Sin[kStatesInLds ? D : 1][D + 8];
  T Zin[kStatesInLds ? D : 1][D + 8];
  T phi[SPM][D + 8];
  T psi[CH][D + 8];
  T dy[CH][D + 8];
  T deltaT[SPM][D + 8];
  T QT[SPM][CH + 8];       // Q^T[s][q],  Q[q][s] = Ws[s, q-1] (psi_q . phi_s)
  T Qp[CH][SPM + 8];       // Q'[q][s] = Ws[s, q-1] (dy_q . delta_s)
  T QpT[SPM][CH + 8];
  T dD[D][SPM + 8];        // dDelta[i][s]
  T wsh[CH][SPM + 8];      // Ws[s, tau-1]
  float Lm[CH][SPM + 1];   // (dy_q . delta_s)(psi_q . phi_s)
  float LWs[CH][CH + 1], LWz[CH][CH + 1];
  ChunkScalars<CH> sc;
  float hS[SPM], hZ[SPM], fS[CH], fZ[CH];
  float HWsS[CH], HWzS[CH], HWzZ[CH];
  float A1[CH + 1], K1[CH + 1], B1[CH + 1];
  float gram[4];
  float red[kSegWaves][4];
  // followed by the halo carry: float carry[2][H][2 * D] (dynamic size)
};

template <typename T>
__device__ __forceinline__ float src_w(int gate_mode, float ug, const float* wl, int e, int t, int j) {
  return gate_mode == GATE_TOKEN ? ug : (gate_mode == GATE_LAG ? wl[t * e + j] : 1.f);
}

template <typename T, int CH, int D>
__global__ __launch_bounds__(kSegThreads) void k_bwd_seg(const Geom g, const BwdPtrs<T> a, const SegGeom sg,
                                                           const BwdSegPtrs p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  typedef BwdSegSmem<T, CH, D> Sm;
  constexpr int SPM = Sm::SPM;
  constexpr bool SIL = Sm::kStatesInLds;
  constexpr int NTD = D / 16;
  constexpr int NT2 = (NTD * NTD + kSegWaves - 1) / kSegWaves;   // owned state tiles per wave
  typedef MM<T> M;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int seg = blockIdx.x, bh = blockIdx.y;
  const int H = g.H, SP = g.SP, e = g.e;
  const size_t tb = (size_t)bh * g.T;
  const size_t sb = (size_t)bh * D * D;
  const int c_begin = seg * sg.G, c_end = min(g.nc, c_begin + sg.G);
  // the segment's last H tokens: their partial (dv, dphi) goes to tail_part (merged by the fixup with the
  // next segment's halo and the d buffer_out terms)
  const int seg_tail0 = min(g.T, c_end * g.Lc) - H;
  float* rw = p.rw + ((size_t)bh * sg.nseg + seg) * (size_t)sg.G * 2 * D * D;

  // ---- 1. adjoint at the segment end (owned tiles: wave + 8 j)
  float dS[NT2][4], dZ[NT2][4], dsr[NT2][4];
#pragma unroll
  for (int j = 0; j < NT2; ++j) {
    const int tile = wave + kSegWaves * j;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      dS[j][r] = 0.f; dZ[j][r] = 0.f; dsr[j][r] = 0.f;
      if (tile < NTD * NTD) {
        const int i = (tile / NTD) * 16 + 4 * (lane >> 4) + r, k = (tile % NTD) * 16 + (lane & 15);
        const size_t off = sb + (size_t)i * D + k;
        float ds = a.dS_T ? a.dS_T[off] : 0.f;
        if (g.clamp_final) ds *= clamp_mask(p.final_raw[off]);
        dS[j][r] = ds;
        dZ[j][r] = (g.momentum && a.dZ_T) ? a.dZ_T[off] : 0.f;
      }
    }
  }
  for (int js = sg.nseg - 1; js > seg; --js) {
    const float* ag = p.adj_agg + ((size_t)bh * sg.nseg + js) * sg.agg_stride;
    const float ta = ag[2 * D * D], tk = ag[2 * D * D + 1], tbb = ag[2 * D * D + 2];
#pragma unroll
    for (int j = 0; j < NT2; ++j) {
      const int tile = wave + kSegWaves * j;
      if (tile >= NTD * NTD) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = (tile / NTD) * 16 + 4 * (lane >> 4) + r, k = (tile % NTD) * 16 + (lane & 15);
        const float Lv = ag[(size_t)i * D + k], Kv = ag[(size_t)D * D + (size_t)i * D + k];
        const float s_out = dS[j][r];
        dS[j][r] = ta * s_out + Lv;
        dZ[j][r] = g.momentum ? (tbb * dZ[j][r] - tk * s_out + Kv) : 0.f;
      }
    }
  }

  // ---- 2. forward re-walk of the segment -> raw chunk-start states in rw
  {
    FwdPtrs<T> fa;
    fa.k = a.k; fa.q = a.q; fa.v = a.v; fa.lr = a.lr; fa.decay = a.decay; fa.beta = a.beta; fa.gate = a.gate;
    fa.S_ref = a.S_ref; fa.S0 = a.S0; fa.Z0 = a.Z0; fa.buf_in = a.buf_in;
    fa.y = nullptr; fa.S_T = nullptr; fa.Z_T = nullptr; fa.buf_out = nullptr; fa.saved = nullptr;
    fwd_segment<T, CH, D, WALK_REWALK>(g, fa, sg, nullptr, const_cast<float*>(p.seg_states), rw, nullptr, smem_raw);
  }
  __syncthreads();

  Sm& sm = *reinterpret_cast<Sm*>(smem_raw);
  float* carry = reinterpret_cast<float*>(smem_raw + sizeof(Sm));   // [2][H][2D]
  for (int idx = tid; idx < D * D; idx += kSegThreads) sm.sref[idx / D][idx % D] = from_f32<T>(a.S_ref[sb + idx]);
  for (int idx = tid; idx < 2 * H * 2 * D; idx += kSegThreads) carry[idx] = 0.f;

  // ---- 3. reverse walk
  for (int c = c_end - 1; c >= c_begin; --c) {
    const int jc = c - c_begin;
    const int t0 = c * g.Lc, t1 = min(g.T, t0 + g.Lc), L = t1 - t0;
    const bool bufchunk = (c == 0) && g.has_buf;
    const bool clamp_in = (c > 0) && clamp_after(g, t0);
    const bool first = c == c_begin, last = c == c_end - 1;
    const float* Sin_g = rw + (size_t)jc * 2 * D * D;   // raw
    const float* Zin_g = Sin_g + (size_t)D * D;
    float* cur_carry = carry + (size_t)(c & 1) * H * 2 * D;        // this chunk's halo -> chunk c-1
    float* prev_carry = carry + (size_t)((c + 1) & 1) * H * 2 * D; // chunk c+1's halo -> this chunk's tail
    __syncthreads();

    // ---- loads
    for (int idx = tid; idx < SP * (D / 8); idx += kSegThreads) {
      const int s = idx / (D / 8), c8 = idx % (D / 8);
      const int pp = t0 - H + s;
      Vec8<T> x = (s < H + L && pp >= 0) ? vec8_load(a.k + (tb + pp) * D + c8 * 8) : Vec8<T>::zero();
      if (g.map_mode == MAP_ELEMENTWISE) x = x.mapped(g.map_deg);
      x.store(&sm.phi[s][c8 * 8]);
    }
    for (int idx = tid; idx < CH * (D / 8); idx += kSegThreads) {
      const int t = idx / (D / 8), c8 = idx % (D / 8);
      Vec8<T> x = t < L ? vec8_load(a.q + (tb + t0 + t) * D + c8 * 8) : Vec8<T>::zero();
      if (g.map_mode == MAP_ELEMENTWISE) x = x.mapped(g.map_deg);
      x.store(&sm.psi[t][c8 * 8]);
      const Vec8<T> dv = (t < L && a.dy) ? vec8_load(a.dy + (tb + t0 + t) * D + c8 * 8) : Vec8<T>::zero();
      dv.store(&sm.dy[t][c8 * 8]);
    }
    if (tid < CH) {
      const bool in = tid < L;
      sm.sc.alpha[tid] = in ? to_f32(a.decay[tb + t0 + tid]) : 1.f;
      sm.sc.eta[tid] = in ? to_f32(a.lr[tb + t0 + tid]) : 0.f;
      sm.sc.beta[tid] = in ? (g.momentum ? to_f32(a.beta[tb + t0 + tid]) : 0.f) : 1.f;
      sm.fS[tid] = 0.f; sm.fZ[tid] = 0.f;
    }
    for (int s = tid; s < SPM; s += kSegThreads) { sm.hS[s] = 0.f; sm.hZ[s] = 0.f; }
    if (g.gate_mode == GATE_TOKEN) {
      for (int s = tid; s < SP; s += kSegThreads) {
        const int pp = t0 - H + s;
        sm.sc.ug[s] = (s < H + L) ? (pp >= 0 ? to_f32(a.gate[tb + pp]) : 1.f) : 0.f;
      }
    } else if (g.gate_mode == GATE_LAG) {
      for (int idx = tid; idx < CH * e; idx += kSegThreads) {
        const int t = idx / e;
        sm.sc.wl[idx] = (t < L) ? to_f32(a.gate[(tb + t0) * e + idx]) : 0.f;
      }
    }
    // states: carried adjoint (registers) and the re-walk's chunk-start state -> LDS operands, Grams
    {
      float gss = 0.f, gsz = 0.f, gzz = 0.f;
#pragma unroll
      for (int j = 0; j < NT2; ++j) {
        const int tile = wave + kSegWaves * j;
        if (tile >= NTD * NTD) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = (tile / NTD) * 16 + 4 * (lane >> 4) + r, k = (tile % NTD) * 16 + (lane & 15);
          float s_in = Sin_g[(size_t)i * D + k];
          if (clamp_in) s_in = clamp100(s_in);
          const float z_in = g.momentum ? Zin_g[(size_t)i * D + k] : 0.f;
          gss += dS[j][r] * s_in; gsz += dS[j][r] * z_in; gzz += dZ[j][r] * z_in;
          sm.dSe[i][k] = from_f32<T>(dS[j][r]);
          sm.dZe[i][k] = from_f32<T>(dZ[j][r]);
          if constexpr (SIL) {
            sm.Sin[i][k] = from_f32<T>(s_in);
            sm.Zin[i][k] = from_f32<T>(z_in);
          }
        }
      }
      for (int off = 32; off > 0; off >>= 1) {
        gss += __shfl_xor(gss, off); gsz += __shfl_xor(gsz, off); gzz += __shfl_xor(gzz, off);
      }
      if (lane == 0) { sm.red[wave][0] = gss; sm.red[wave][1] = gsz; sm.red[wave][2] = gzz; }
    }
    __syncthreads();
    if (tid == 0) {
      for (int q = 0; q < 3; ++q) {
        float s = 0.f;
        for (int w = 0; w < kSegWaves; ++w) s += sm.red[w][q];
        sm.gram[q] = s;
      }
    }
    if (bufchunk) {   // <dS_end, B_s>, <dZ_end, B_s> for the dense buffer sources
      for (int s = 0; s < H; ++s) {
        const float* Bs = a.buf_in + ((size_t)bh * H + s) * D * D;
        float hs = 0.f, hz = 0.f;
#pragma unroll
        for (int j = 0; j < NT2; ++j) {
          const int tile = wave + kSegWaves * j;
          if (tile >= NTD * NTD) continue;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = (tile / NTD) * 16 + 4 * (lane >> 4) + r, k = (tile % NTD) * 16 + (lane & 15);
            const float b = Bs[(size_t)i * D + k];
            hs += dS[j][r] * b; hz += dZ[j][r] * b;
          }
        }
        for (int off = 32; off > 0; off >>= 1) { hs += __shfl_xor(hs, off); hz += __shfl_xor(hz, off); }
        if (lane == 0) { atomicAdd(&sm.hS[s], hs); atomicAdd(&sm.hZ[s], hz); }
      }
    }

    // ---- phase A: G1 delta^T (waves 0-5) | coefficients (waves 6-7)
    if (wave < 6) {
      for (int tile = wave; tile < (SP / 16) * NTD; tile += 6) {
        const int m0 = (tile / NTD) * 16, n0 = (tile % NTD) * 16;
        f32x4 acc = zero4();
#pragma unroll
        for (int k0 = 0; k0 < D; k0 += M::KS)
          acc = M::mma(frag_ld_row<T>(&sm.phi[0][0], D + 8, m0, k0), frag_ld_row<T>(&sm.sref[0][0], D + 8, n0, k0), acc);
        const int i = n0 + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int s = m0 + 4 * (lane >> 4) + r;
          const int pp = t0 - H + s;
          float d = 0.f;
          if (s < H + L && pp >= 0) d = acc[r] - to_f32(a.v[(tb + pp) * D + i]);
          sm.deltaT[s][i] = from_f32<T>(d);
        }
      }
    } else {
      const int ci = tid - 6 * kWave;
      // per-source recurrences (Ws[s, tau-1] -> wsh, end values) and a / kappa / b with the shifted arrays
      const float* __restrict__ al = sm.sc.alpha;
      const float* __restrict__ et = sm.sc.eta;
      const float* __restrict__ be = sm.sc.beta;
      const float* __restrict__ wl = sm.sc.wl;
      if (ci < SP) {
        const int s = ci;
        const float us = g.gate_mode == GATE_TOKEN ? sm.sc.ug[s] : 1.f;
        float ws = 0.f, wz = 0.f;
        for (int t = 0; t < CH; ++t) {
          sm.wsh[t][s] = from_f32<T>(ws);
          const int j = t + H - s;
          float w = 0.f;
          if (j >= 0 && j < e && t < L) w = (g.gate_mode == GATE_LAG) ? wl[t * e + j] : us;
          wz = be[t] * wz + w;
          ws = al[t] * ws + et[t] * wz;
        }
        sm.sc.wsend[s] = ws;
        sm.sc.wzend[s] = wz;
      } else if (ci == 127) {
        float ac = 1.f, kc = 0.f, bc = 1.f;
        sm.A1[0] = 1.f; sm.K1[0] = 0.f; sm.B1[0] = 1.f;
        for (int t = 0; t < CH; ++t) {
          sm.sc.acoef[t] = ac; sm.sc.kcoef[t] = kc;
          bc = be[t] * bc; ac = al[t] * ac; kc = al[t] * kc + et[t] * bc;
          sm.A1[t + 1] = ac; sm.K1[t + 1] = kc; sm.B1[t + 1] = bc;
        }
        sm.sc.endc[0] = ac; sm.sc.endc[1] = kc; sm.sc.endc[2] = bc;
      }
    }
    __syncthreads();
    // G2 / G3: Kmat = psi phi^T, K3 = dy delta -> Q^T, Q', Q'^T, Lm
    {
      const int nts = SP / 16;
      for (int tile = wave; tile < (CH / 16) * nts; tile += kSegWaves) {
        const int m0 = (tile / nts) * 16, n0 = (tile % nts) * 16;
        f32x4 kk = zero4(), k3 = zero4();
#pragma unroll
        for (int k0 = 0; k0 < D; k0 += M::KS) {
          kk = M::mma(frag_ld_row<T>(&sm.psi[0][0], D + 8, m0, k0), frag_ld_row<T>(&sm.phi[0][0], D + 8, n0, k0), kk);
          k3 = M::mma(frag_ld_row<T>(&sm.dy[0][0], D + 8, m0, k0), frag_ld_row<T>(&sm.deltaT[0][0], D + 8, n0, k0), k3);
        }
        const int s = n0 + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = m0 + 4 * (lane >> 4) + r;
          const float w = to_f32(sm.wsh[t][s]);
          sm.QT[s][t] = from_f32<T>(w * kk[r]);
          const T qp = from_f32<T>(w * k3[r]);
          sm.Qp[t][s] = qp;
          sm.QpT[s][t] = qp;
          sm.Lm[t][s] = kk[r] * k3[r];
        }
      }
    }
    __syncthreads();

    // ---- phase B: G4  dDelta[i, s] = Wz_end[s] (dZ_end phi_s)_i - Ws_end[s] (dS_end phi_s)_i - sum_q dy_q[i] Q[q, s]
    {
      const int nts = SP / 16;
      for (int tile = wave; tile < NTD * nts; tile += kSegWaves) {
        const int m0 = (tile / nts) * 16, n0 = (tile % nts) * 16;
        f32x4 az = zero4(), as = zero4(), aq = zero4();
#pragma unroll
        for (int k0 = 0; k0 < D; k0 += M::KS) {
          const typename M::frag fb = frag_ld_row<T>(&sm.phi[0][0], D + 8, n0, k0);
          as = M::mma(frag_ld_row<T>(&sm.dSe[0][0], D + 8, m0, k0), fb, as);
          az = M::mma(frag_ld_row<T>(&sm.dZe[0][0], D + 8, m0, k0), fb, az);
        }
        for (int k0 = 0; k0 < CH; k0 += M::KS)
          aq = M::mma(frag_ld<T>(&sm.dy[0][0], 1, D + 8, m0, k0), frag_ld_row<T>(&sm.QT[0][0], CH + 8, n0, k0), aq);
        const int s = n0 + (lane & 15);
        const float wz = sm.sc.wzend[s], ws = sm.sc.wsend[s];
        float hs = 0.f, hz = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = m0 + 4 * (lane >> 4) + r;
          const float d = to_f32(sm.deltaT[s][i]);
          hs += d * as[r];
          hz += d * az[r];
          sm.dD[i][s] = from_f32<T>(wz * az[r] - ws * as[r] - aq[r]);
        }
        hs += __shfl_xor(hs, 16); hs += __shfl_xor(hs, 32);
        hz += __shfl_xor(hz, 16); hz += __shfl_xor(hz, 32);
        if (lane < 16) { atomicAdd(&sm.hS[s], hs); atomicAdd(&sm.hZ[s], hz); }
      }
    }
    __syncthreads();

    // ---- phase C: dv from dDelta; G6 dS_ref; G7 dpsi (+ fS, fZ); d buffer_in
    {
      const int tail0 = t1 - H;
      for (int idx = tid; idx < (H + L) * D; idx += kSegThreads) {
        const int s = idx / D, i = idx % D;
        const int pp = t0 - H + s;
        if (pp < 0) continue;
        float val = -to_f32(sm.dD[i][s]);
        if (s < H) {
          if (first) { if (c > 0) p.halo_part[(((size_t)bh * sg.nseg + seg) * H + s) * (2 * D) + i] = val; }
          else cur_carry[s * 2 * D + i] = val;
          continue;
        }
        if (pp >= tail0) val += prev_carry[(pp - tail0) * 2 * D + i];
        if (pp >= seg_tail0) p.tail_part[(((size_t)bh * sg.nseg + seg) * H + (pp - seg_tail0)) * (2 * D) + i] = val;
        else a.dv[(tb + pp) * D + i] = from_f32<T>(val);
      }
    }
#pragma unroll
    for (int j = 0; j < NT2; ++j) {   // G6: dS_ref[i, k] += sum_s dDelta[i, s] phi_s[k]
      const int tile = wave + kSegWaves * j;
      if (tile >= NTD * NTD) continue;
      const int m0 = (tile / NTD) * 16, n0 = (tile % NTD) * 16;
      f32x4 acc = zero4();
      for (int k0 = 0; k0 < SP; k0 += M::KS)
        acc = M::mma(frag_ld_row<T>(&sm.dD[0][0], SPM + 8, m0, k0), frag_ld<T>(&sm.phi[0][0], 1, D + 8, n0, k0), acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) dsr[j][r] += acc[r];
    }
    for (int tile = wave; tile < (CH / 16) * NTD; tile += kSegWaves) {   // G7
      const int m0 = (tile / NTD) * 16, n0 = (tile % NTD) * 16;
      f32x4 as = zero4(), az = zero4(), aq = zero4();
#pragma unroll
      for (int k0 = 0; k0 < D; k0 += M::KS) {
        const typename M::frag fa = frag_ld_row<T>(&sm.dy[0][0], D + 8, m0, k0);
        if constexpr (SIL) {
          as = M::mma(fa, frag_ld<T>(&sm.Sin[0][0], 1, D + 8, n0, k0), as);
          az = M::mma(fa, frag_ld<T>(&sm.Zin[0][0], 1, D + 8, n0, k0), az);
        } else {
          typename M::frag fs;
          {
            const int kb = k0 + (lane >> 4) * M::KL;
            const float* q = Sin_g + (size_t)kb * D + n0 + (lane & 15);
            if constexpr (M::KL == 1) fs = static_cast<T>(clamp_in ? clamp100(q[0]) : q[0]);
            else {
#pragma unroll
              for (int ee = 0; ee < M::KL; ++ee) {
                const float x = q[(size_t)ee * D];
                fs[ee] = static_cast<T>(clamp_in ? clamp100(x) : x);
              }
            }
          }
          as = M::mma(fa, fs, as);
          az = M::mma(fa, frag_ld_or_zero<T>(g.momentum ? Zin_g : nullptr, 1, D, n0, k0), az);
        }
      }
      for (int k0 = 0; k0 < SP; k0 += M::KS)
        aq = M::mma(frag_ld_row<T>(&sm.Qp[0][0], SPM + 8, m0, k0), frag_ld<T>(&sm.phi[0][0], 1, D + 8, n0, k0), aq);
      const int k = n0 + (lane & 15);
      f32x4 dpsi;
      float fsp[4], fzp[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = m0 + 4 * (lane >> 4) + r;
        dpsi[r] = sm.A1[t] * as[r] - sm.K1[t] * az[r] - aq[r];
        const float ps = to_f32(sm.psi[t][k]);
        fsp[r] = as[r] * ps;
        fzp[r] = az[r] * ps;
      }
      if (bufchunk) {
        for (int s = 0; s < H; ++s) {
          const float* Bs = a.buf_in + ((size_t)bh * H + s) * D * D;
          f32x4 ab = zero4();
#pragma unroll
          for (int k0 = 0; k0 < D; k0 += M::KS)
            ab = M::mma(frag_ld_row<T>(&sm.dy[0][0], D + 8, m0, k0), frag_ld<T>(Bs, 1, D, n0, k0), ab);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = m0 + 4 * (lane >> 4) + r;
            dpsi[r] -= to_f32(sm.wsh[t][s]) * ab[r];
            float lm = ab[r] * to_f32(sm.psi[t][k]);
            for (int off = 8; off > 0; off >>= 1) lm += __shfl_xor(lm, off);
            if ((lane & 15) == 0) atomicAdd(&sm.Lm[t][s], lm);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = m0 + 4 * (lane >> 4) + r;
        float fsv = fsp[r], fzv = fzp[r];
        for (int off = 8; off > 0; off >>= 1) { fsv += __shfl_xor(fsv, off); fzv += __shfl_xor(fzv, off); }
        if ((lane & 15) == 0) { atomicAdd(&sm.fS[t], fsv); atomicAdd(&sm.fZ[t], fzv); }
        if (t < L) {
          float outv = dpsi[r];
          if (g.map_mode == MAP_ELEMENTWISE) outv *= poly_map_grad(to_f32(a.q[(tb + t0 + t) * D + k]), g.map_deg);
          a.dq[(tb + t0 + t) * D + k] = from_f32<T>(outv);
        }
      }
    }
    if (bufchunk) {   // d buffer_in[s] = Wz_end[s] dZ_end - Ws_end[s] dS_end - sum_q Ws[s, q-1] dy_q psi_q^T
      for (int s = 0; s < H; ++s) {
        float* dst = a.dbuf_in + ((size_t)bh * H + s) * D * D;
#pragma unroll
        for (int j = 0; j < NT2; ++j) {
          const int tile = wave + kSegWaves * j;
          if (tile >= NTD * NTD) continue;
          const int m0 = (tile / NTD) * 16, n0 = (tile % NTD) * 16;
          f32x4 acc = zero4();
          for (int k0 = 0; k0 < CH; k0 += M::KS) {
            typename M::frag fa;
            const int qb = k0 + (lane >> 4) * M::KL;
            const int i = m0 + (lane & 15);
            if constexpr (M::KL == 1) fa = static_cast<T>(to_f32(sm.dy[qb][i]) * to_f32(sm.wsh[qb][s]));
            else {
#pragma unroll
              for (int ee = 0; ee < M::KL; ++ee)
                fa[ee] = static_cast<T>(to_f32(sm.dy[qb + ee][i]) * to_f32(sm.wsh[qb + ee][s]));
            }
            acc = M::mma(fa, frag_ld<T>(&sm.psi[0][0], 1, D + 8, n0, k0), acc);
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = m0 + 4 * (lane >> 4) + r, k = n0 + (lane & 15);
            dst[(size_t)i * D + k] = sm.sc.wzend[s] * dZ[j][r] - sm.sc.wsend[s] * dS[j][r] - acc[r];
          }
        }
      }
    }
    __syncthreads();

    // ---- phase D: G5  dphi[s, k] = Wz_end dZ_end^T delta_s - Ws_end dS_end^T delta_s - sum_q Q'[q, s] psi_q + S_ref^T dDelta_s
    {
      const int tail0 = t1 - H;
      for (int tile = wave; tile < (SP / 16) * NTD; tile += kSegWaves) {
        const int m0 = (tile / NTD) * 16, n0 = (tile % NTD) * 16;
        f32x4 a1 = zero4(), a2 = zero4(), a3 = zero4(), a4 = zero4();
#pragma unroll
        for (int k0 = 0; k0 < D; k0 += M::KS) {
          const typename M::frag fa = frag_ld_row<T>(&sm.deltaT[0][0], D + 8, m0, k0);
          a1 = M::mma(fa, frag_ld<T>(&sm.dZe[0][0], 1, D + 8, n0, k0), a1);
          a2 = M::mma(fa, frag_ld<T>(&sm.dSe[0][0], 1, D + 8, n0, k0), a2);
          a4 = M::mma(frag_ld<T>(&sm.dD[0][0], 1, SPM + 8, m0, k0), frag_ld<T>(&sm.sref[0][0], 1, D + 8, n0, k0), a4);
        }
        for (int k0 = 0; k0 < CH; k0 += M::KS)
          a3 = M::mma(frag_ld_row<T>(&sm.QpT[0][0], CH + 8, m0, k0), frag_ld<T>(&sm.psi[0][0], 1, D + 8, n0, k0), a3);
        const int k = n0 + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int s = m0 + 4 * (lane >> 4) + r;
          const int pp = t0 - H + s;
          if (s >= H + L || pp < 0) continue;
          float val = sm.sc.wzend[s] * a1[r] - sm.sc.wsend[s] * a2[r] - a3[r] + a4[r];
          if (s < H) {
            if (first) { if (c > 0) p.halo_part[(((size_t)bh * sg.nseg + seg) * H + s) * (2 * D) + D + k] = val; }
            else cur_carry[s * 2 * D + D + k] = val;
            continue;
          }
          if (pp >= tail0) val += prev_carry[(pp - tail0) * 2 * D + D + k];
          if (pp >= seg_tail0) {
            p.tail_part[(((size_t)bh * sg.nseg + seg) * H + (pp - seg_tail0)) * (2 * D) + D + k] = val;
          } else {
            if (g.map_mode == MAP_ELEMENTWISE) val *= poly_map_grad(to_f32(a.k[(tb + pp) * D + k]), g.map_deg);
            a.dk[(tb + pp) * D + k] = from_f32<T>(val);
          }
        }
      }
    }

    // ---- phase E: chunk-start adjoint (the B1 step) -> carried (dS, dZ) for chunk c - 1
    {
      const float ae = sm.sc.endc[0], ke = sm.sc.endc[1], be = sm.sc.endc[2];
#pragma unroll
      for (int j = 0; j < NT2; ++j) {
        const int tile = wave + kSegWaves * j;
        if (tile >= NTD * NTD) continue;
        const int m0 = (tile / NTD) * 16, n0 = (tile % NTD) * 16;
        f32x4 aa = zero4(), ak = zero4();
        for (int k0 = 0; k0 < CH; k0 += M::KS) {
          const typename M::frag fb = frag_ld<T>(&sm.psi[0][0], 1, D + 8, n0, k0);
          aa = M::mma(frag_ld_kscaled<T>(&sm.dy[0][0], 1, D + 8, m0, k0, sm.sc.acoef), fb, aa);
          ak = M::mma(frag_ld_kscaled<T>(&sm.dy[0][0], 1, D + 8, m0, k0, sm.sc.kcoef), fb, ak);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = m0 + 4 * (lane >> 4) + r, k = n0 + (lane & 15);
          const float lam = ae * dS[j][r] + aa[r];
          const float mu = g.momentum ? (be * dZ[j][r] - ke * dS[j][r] - ak[r]) : 0.f;
          const float mk = clamp_in ? clamp_mask(Sin_g[(size_t)i * D + k]) : 1.f;
          dS[j][r] = lam * mk;
          dZ[j][r] = mu;
          if (c == 0) {
            a.dS0[sb + (size_t)i * D + k] = lam;
            if (g.momentum && a.dZ0) a.dZ0[sb + (size_t)i * D + k] = mu;
          }
        }
      }
    }

    // ---- phase F: scalar gradients
    if (tid < CH) {
      const int q = tid;
      float lz = 0.f, ls = 0.f;
      for (int t = 0; t < CH; ++t) {
        float acc = 0.f;
        for (int j = 0; j < e && t < L; ++j) {
          const int s = t + H - j;
          acc += src_w<T>(g.gate_mode, sm.sc.ug[s], sm.sc.wl, e, t, j) * sm.Lm[q][s];
        }
        lz = sm.sc.beta[t] * lz + acc;
        ls = sm.sc.alpha[t] * ls + sm.sc.eta[t] * lz;
        sm.LWs[q][t] = ls;
        sm.LWz[q][t] = lz;
      }
    } else if (tid == CH) {
      float hzs = 0.f, hss = 0.f, hzz = 0.f;
      for (int t = 0; t < CH; ++t) {
        float as = 0.f, az = 0.f;
        for (int j = 0; j < e && t < L; ++j) {
          const int s = t + H - j;
          const float w = src_w<T>(g.gate_mode, sm.sc.ug[s], sm.sc.wl, e, t, j);
          as += w * sm.hS[s];
          az += w * sm.hZ[s];
        }
        hzs = sm.sc.beta[t] * hzs + as;
        hss = sm.sc.alpha[t] * hss + sm.sc.eta[t] * hzs;
        hzz = sm.sc.beta[t] * hzz + az;
        sm.HWsS[t] = hss; sm.HWzS[t] = hzs; sm.HWzZ[t] = hzz;
      }
    }
    __syncthreads();
    // one thread per (target t, term): term 0 -> dalpha, 1 -> deta, 2 -> dbeta, 3 + j -> dw[t, j]
    {
      const int nterm = 3 + (g.gate_mode != GATE_NONE ? e : 0);
      for (int idx = tid; idx < L * nterm; idx += kSegThreads) {
        const int t = idx % L, term = idx / L;
        const float gss = sm.gram[0], gsz = sm.gram[1], gzz = sm.gram[2];
        const float am1 = sm.A1[t], km1 = sm.K1[t], bm1 = sm.B1[t];
        const float b0 = sm.B1[t + 1];
        float acc = 0.f;
        float Ar = 1.f, Br = 1.f, Mr = sm.sc.eta[t];
        const int sj = term >= 3 ? t + H - (term - 3) : 0;
        for (int q = t + 1; q < L; ++q) {
          float v;
          if (term == 0) {
            const float LWs_m1 = t > 0 ? sm.LWs[q][t - 1] : 0.f;
            v = Ar * (am1 * sm.fS[q] - km1 * sm.fZ[q] - LWs_m1);
          } else if (term == 1) {
            v = Ar * (b0 * sm.fZ[q] + sm.LWz[q][t]);
          } else if (term == 2) {
            const float LWz_m1 = t > 0 ? sm.LWz[q][t - 1] : 0.f;
            v = Mr * (bm1 * sm.fZ[q] + LWz_m1);
          } else {
            v = Mr * sm.Lm[q][sj];
          }
          acc += v;
          Ar *= sm.sc.alpha[q];
          Br *= sm.sc.beta[q];
          Mr = sm.sc.alpha[q] * Mr + sm.sc.eta[q] * Br;
        }
        const size_t tt = tb + t0 + t;
        if (term == 0) {
          const float HWsS_m1 = t > 0 ? sm.HWsS[t - 1] : 0.f;
          a.ddecay[tt] = from_f32<T>(acc + Ar * (am1 * gss - km1 * gsz - HWsS_m1));
        } else if (term == 1) {
          a.dlr[tt] = from_f32<T>(-(acc + Ar * (b0 * gsz + sm.HWzS[t])));
        } else if (term == 2) {
          if (g.momentum && a.dbeta) {
            const float HWzS_m1 = t > 0 ? sm.HWzS[t - 1] : 0.f;
            const float HWzZ_m1 = t > 0 ? sm.HWzZ[t - 1] : 0.f;
            a.dbeta[tt] = from_f32<T>(Br * (bm1 * gzz + HWzZ_m1) - Mr * (bm1 * gsz + HWzS_m1) - acc);
          }
        } else {
          const int j = term - 3;
          const float v = Br * sm.hZ[sj] - Mr * sm.hS[sj] - acc;
          if (g.gate_mode == GATE_LAG) a.dgate[tt * e + j] = from_f32<T>(v);
          else p.dw[tt * e + j] = v;
        }
      }
    }
  }

  // ---- 4. segment outputs: dS_ref partial
  float* dst = p.dsref_part + ((size_t)bh * sg.nseg + seg) * D * D;
#pragma unroll
  for (int j = 0; j < NT2; ++j) {
    const int tile = wave + kSegWaves * j;
    if (tile >= NTD * NTD) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = (tile / NTD) * 16 + 4 * (lane >> 4) + r, k = (tile % NTD) * 16 + (lane & 15);
      dst[(size_t)i * D + k] = dsr[j][r];
    }
  }
}

// ---------------------------------------------------------------------------------------------
// segment-boundary fixup: grid (nseg, BH)
// ---------------------------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(kThreads) void k_bwd_seg_fixup(const Geom g, const BwdPtrs<T> a, const SegGeom sg,
                                                              const BwdSegPtrs p) {
  __shared__ float sphi[D], sdel[D], sdd[D], sdb[D];
  const int seg = blockIdx.x, bh = blockIdx.y;
  const int H = g.H, e = g.e;
  const int c_begin = seg * sg.G, c_end = min(g.nc, c_begin + sg.G);
  const int tok0 = c_begin * g.Lc, tok1 = min(g.T, c_end * g.Lc);
  const size_t tb = (size_t)bh * g.T;
  const int tid = threadIdx.x;
  // token-gate gradient du_p = sum_j dw[p + j, j] (the d buffer_out term is added below)
  if (g.gate_mode == GATE_TOKEN) {
    for (int pp = tok0 + tid; pp < tok1; pp += kThreads) {
      if (a.dbuf_out && pp >= g.T - H) continue;
      float du = 0.f;
      for (int j = 0; j < e && pp + j < g.T; ++j) du += p.dw[(tb + pp + j) * e + j];
      a.dgate[tb + pp] = from_f32<T>(du);
    }
  }
  if (H == 0) return;
  const int tail0 = tok1 - H;
  const bool has_next = seg + 1 < sg.nseg;
  for (int h = 0; h < H; ++h) {
    const int pp = tail0 + h;
    if (pp < tok0) continue;                       // token of the previous segment (short last segment)
    const size_t tp = (((size_t)bh * sg.nseg + seg) * H + h) * (2 * D);
    const size_t hp = has_next ? (((size_t)bh * sg.nseg + seg + 1) * H + h) * (2 * D) : 0;
    const bool outbuf = (a.dbuf_out != nullptr) && (pp >= g.T - H);
    const int kb = pp - (g.T - H);
    __syncthreads();
    if (outbuf) {
      for (int k = tid; k < D; k += kThreads) sphi[k] = ld_map(a.k, (tb + pp) * D + k, g.map_mode, g.map_deg);
      __syncthreads();
      const float cp = (g.gate_mode == GATE_TOKEN) ? to_f32(a.gate[tb + pp]) : 1.f;
      const float* dB = a.dbuf_out + ((size_t)bh * H + kb) * D * D;
      const float* Sr = a.S_ref + (size_t)bh * D * D;
      for (int i = tid; i < D; i += kThreads) {
        float acc = 0.f, accd = 0.f;
        for (int k = 0; k < D; ++k) { acc += Sr[(size_t)i * D + k] * sphi[k]; accd += dB[(size_t)i * D + k] * sphi[k]; }
        sdel[i] = acc - to_f32(a.v[(tb + pp) * D + i]);
        sdb[i] = accd;
        sdd[i] = cp * accd;
      }
      __syncthreads();
      if (tid == 0 && g.gate_mode == GATE_TOKEN) {
        float du = 0.f;
        for (int i = 0; i < D; ++i) du += sdel[i] * sdb[i];
        for (int j = 0; j < e && pp + j < g.T; ++j) du += p.dw[(tb + pp + j) * e + j];
        a.dgate[tb + pp] = from_f32<T>(du);
      }
      float* dsr = p.dsref_part + ((size_t)bh * sg.nseg + seg) * D * D;
      for (int idx = tid; idx < D * D; idx += kThreads) dsr[idx] += sdd[idx / D] * sphi[idx % D];
    }
    for (int i = tid; i < D; i += kThreads) {
      float val = p.tail_part[tp + i] + (has_next ? p.halo_part[hp + i] : 0.f);
      if (outbuf) val -= sdd[i];
      a.dv[(tb + pp) * D + i] = from_f32<T>(val);
    }
    for (int k = tid; k < D; k += kThreads) {
      float val = p.tail_part[tp + D + k] + (has_next ? p.halo_part[hp + D + k] : 0.f);
      if (outbuf) {
        const float cp = (g.gate_mode == GATE_TOKEN) ? to_f32(a.gate[tb + pp]) : 1.f;
        const float* dB = a.dbuf_out + ((size_t)bh * H + kb) * D * D;
        const float* Sr = a.S_ref + (size_t)bh * D * D;
        float acc = 0.f;
        for (int i = 0; i < D; ++i) acc += cp * dB[(size_t)i * D + k] * sdel[i] + Sr[(size_t)i * D + k] * sdd[i];
        val += acc;
      }
      if (g.map_mode == MAP_ELEMENTWISE) val *= poly_map_grad(to_f32(a.k[(tb + pp) * D + k]), g.map_deg);
      a.dk[(tb + pp) * D + k] = from_f32<T>(val);
    }
  }
  // buffer pass-through when T < e - 1: buffer_out[k'] = buffer_in[T + k']
  if (seg == 0 && a.dbuf_out && a.dbuf_in && g.T < H) {
    __syncthreads();
    for (int kq = 0; kq + g.T < H; ++kq) {
      const float* src = a.dbuf_out + ((size_t)bh * H + kq) * D * D;
      float* dstb = a.dbuf_in + ((size_t)bh * H + g.T + kq) * D * D;
      for (int idx = tid; idx < D * D; idx += kThreads) dstb[idx] += src[idx];
    }
  }
}

// dS_ref = sum over segments of the partials.   grid (D*D/256, BH)
__global__ __launch_bounds__(kThreads) void k_seg_reduce_dsref(int nseg, int n, const float* part, float* out) {
  const int bh = blockIdx.y;
  const int idx = blockIdx.x * kThreads + threadIdx.x;
  if (idx >= n) return;
  float acc = 0.f;
  for (int s = 0; s < nseg; ++s) acc += part[((size_t)bh * nseg + s) * n + idx];
  out[(size_t)bh * n + idx] = acc;
}

template <typename T, int CH, int D>
size_t bwd_seg_smem_bytes(int H) {
  const size_t main_sz = sizeof(BwdSegSmem<T, CH, D>) + (size_t)2 * H * 2 * D * sizeof(float);
  const size_t rewalk = sizeof(SegFwdSmem<T, CH, D, false>);
  return main_sz > rewalk ? main_sz : rewalk;
}

template <typename T, int CH, int D>
hipError_t launch_bwd_seg(const Geom& g, const BwdPtrs<T>& a, const SegGeom& sg, const BwdSegPtrs& p,
                          hipStream_t stream) {
  hipError_t err;
  if (sg.nseg > 1) {
    const size_t smem = sizeof(BwdAggSmem<T, CH, D>);
    err = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_bwd_seg_agg<T, CH, D>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (err != hipSuccess) return err;
    prof_begin(KID_BWD_ADJOINT, stream);
    hipLaunchKernelGGL((k_bwd_seg_agg<T, CH, D>), dim3(sg.nseg, g.BH), dim3(kSegThreads), smem, stream, g, a, sg, p);
    prof_end(KID_BWD_ADJOINT, stream);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  {
    const size_t smem = bwd_seg_smem_bytes<T, CH, D>(g.H);
    err = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_bwd_seg<T, CH, D>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (err != hipSuccess) return err;
    prof_begin(KID_BWD_CHUNK, stream);
    hipLaunchKernelGGL((k_bwd_seg<T, CH, D>), dim3(sg.nseg, g.BH), dim3(kSegThreads), smem, stream, g, a, sg, p);
    prof_end(KID_BWD_CHUNK, stream);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  prof_begin(KID_BWD_FIXUP, stream);
  hipLaunchKernelGGL((k_bwd_seg_fixup<T, D>), dim3(sg.nseg, g.BH), dim3(kThreads), 0, stream, g, a, sg, p);
  prof_end(KID_BWD_FIXUP, stream);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  prof_begin(KID_REDUCE_DSREF, stream);
  hipLaunchKernelGGL(k_seg_reduce_dsref, dim3((D * D + kThreads - 1) / kThreads, g.BH), dim3(kThreads), 0, stream,
                     sg.nseg, D * D, (const float*)p.dsref_part, a.dS_ref);
  prof_end(KID_REDUCE_DSREF, stream);
  return hipGetLastError();
}

#define ATLAS_INST_BWD_SEG(T, CH, D)                                                                  \
  template hipError_t launch_bwd_seg<T, CH, D>(const Geom&, const BwdPtrs<T>&, const SegGeom&,        \
                                               const BwdSegPtrs&, hipStream_t);                       \
  template size_t bwd_seg_smem_bytes<T, CH, D>(int);

ATLAS_INST_BWD_SEG(bf16, 32, 64)
ATLAS_INST_BWD_SEG(float, 16, 64)
ATLAS_INST_BWD_SEG(bf16, 32, 32)
ATLAS_INST_BWD_SEG(float, 16, 32)

}  // namespace atlas
