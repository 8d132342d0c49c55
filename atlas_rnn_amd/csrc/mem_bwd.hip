// mem_bwd.hip - backward pass of the chunked memory recurrence (gfx950).
//
// Pass B1 (k_bwd_adjoint_walk): one workgroup per (16 rows, bh) walks the chunks in reverse and
//   carries the adjoint of the chunk-end states (dS_end, dZ_end). Per chunk
//     dS_in = a_end dS_end + sum_tau a_{tau-1} dy_tau psi_tau^T
//     dZ_in = b_end dZ_end - kappa_end dS_end - sum_tau kappa_{tau-1} dy_tau psi_tau^T
//   (the transpose of the forward chunk map; it needs no forward state), with the clamp mask
//   of the forward's raw chunk-end S applied at scan_chunk_len boundaries. Every chunk's
//   (dS_end, dZ_end) is stored.
// Pass B2 (k_bwd_chunk): one workgroup per (chunk, bh), all rows. From the forward's chunk-start
//   states and B1's chunk-end adjoints it forms every gradient of the chunk in closed form:
//     d delta_s = Wz_end[s] dZ_end phi_s - Ws_end[s] dS_end phi_s - sum_q Ws[s,q-1] (psi_q.phi_s) dy_q
//     d phi_s   = Wz_end[s] dZ_end^T delta_s - Ws_end[s] dS_end^T delta_s
//                 - sum_q Ws[s,q-1] (dy_q.delta_s) psi_q + S_ref^T d delta_s
//     d psi_t   = a_{t-1} S_in^T dy_t - kappa_{t-1} Z_in^T dy_t - sum_s Ws[s,t-1] (dy_t.delta_s) phi_s
//     dS_ref   += d delta phi^T,   dv = -d delta
//   and the scalar gradients dalpha_t = <lambda_t, S_{t-1}>, deta_t = -<lambda_t, Z_t>,
//   dbeta_t = <mu_t, Z_{t-1}>, dw[t,j] = <mu_t, delta_{t-j} phi_{t-j}^T> from Gram terms between
//   the forward basis {S_in, Z_in, delta_s phi_s^T} and the adjoint basis {dS_end, dZ_end, dy_q psi_q^T}.
// Pass B3 (k_bwd_fixup): merges the partial (dv, dphi) of tokens whose window spans a chunk
//   boundary, adds the d buffer_out terms, reduces token-gate gradients, applies the feature map
//   derivative. Pass B4 (k_reduce_dsref) sums the per-chunk dS_ref partials.
#include "mem_common.h"
#include "mem_params.h"

namespace atlas {

template <typename T>
__device__ __forceinline__ float ld_map(const T* p, size_t idx, int map_mode, int deg) {
  float x = to_f32(p[idx]);
  return map_mode == MAP_ELEMENTWISE ? poly_map(x, deg) : x;
}

// =============================================================================================
// B1: adjoint walk
// =============================================================================================
template <typename T, int CH, int DK>
struct AdjSmem {
  T psi[CH][DK + 8];
  float dyT[16][CH + 1];
  float alpha[CH], eta[CH], beta[CH];
  float acoef[CH], kcoef[CH];   // a_{tau-1}, kappa_{tau-1}
  float endc[4];
};

template <typename T, int CH, int DK, int DV>
__global__ __launch_bounds__(kThreads) void k_bwd_adjoint_walk(const Geom g, const BwdPtrs<T> a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  typedef AdjSmem<T, CH, DK> Sm;
  Sm& sm = *reinterpret_cast<Sm*>(smem_raw);
  constexpr int NKT = DK / 16;
  constexpr int NOWN = (NKT + kWaves - 1) / kWaves;
  typedef MM<T> M;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int row0 = blockIdx.x * 16;
  const int bh = blockIdx.y;
  const size_t tb = (size_t)bh * g.T;
  const size_t sb = (size_t)bh * DV * DK;
  const size_t cs = (size_t)2 * DV * DK;     // chunk stride of saved / adj

  float dS[NOWN][4], dZ[NOWN][4];
  {
    const size_t last = ((size_t)bh * g.nc + (g.nc - 1)) * cs;
#pragma unroll
    for (int j = 0; j < NOWN; ++j) {
      const int kt = wave + kWaves * j;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        dS[j][r] = 0.f; dZ[j][r] = 0.f;
        if (kt < NKT) {
          const int i = 4 * (lane >> 4) + r, k = kt * 16 + (lane & 15);
          const size_t off = (size_t)(row0 + i) * DK + k;
          float ds = a.dS_T ? a.dS_T[sb + off] : 0.f;
          if (g.clamp_final) ds *= clamp_mask(a.saved[last + off]);
          dS[j][r] = ds;
          dZ[j][r] = (g.momentum && a.dZ_T) ? a.dZ_T[sb + off] : 0.f;
        }
      }
    }
  }

  for (int c = g.nc - 1; c >= 0; --c) {
    const int t0 = c * g.Lc;
    const int t1 = min(g.T, t0 + g.Lc);
    const int L = t1 - t0;
    // store this chunk's end adjoint
#pragma unroll
    for (int j = 0; j < NOWN; ++j) {
      const int kt = wave + kWaves * j;
      if (kt >= NKT) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 4 * (lane >> 4) + r, k = kt * 16 + (lane & 15);
        const size_t so = ((size_t)bh * g.nc + c) * cs + (size_t)(row0 + i) * DK + k;
        a.adj[so] = dS[j][r];
        a.adj[so + (size_t)DV * DK] = dZ[j][r];
      }
    }
    for (int idx = tid; idx < CH * DK; idx += kThreads) {
      const int t = idx / DK, k = idx % DK;
      float val = 0.f;
      if (t < L) val = ld_map(a.q, (tb + t0 + t) * DK + k, g.map_mode, g.map_deg);
      sm.psi[t][k] = from_f32<T>(val);
    }
    for (int idx = tid; idx < 16 * CH; idx += kThreads) {
      const int t = idx / 16, i = idx % 16;
      sm.dyT[i][t] = (t < L && a.dy) ? to_f32(a.dy[(tb + t0 + t) * DV + row0 + i]) : 0.f;
    }
    if (tid < CH) {
      const int t = tid;
      const bool in = t < L;
      sm.alpha[t] = in ? to_f32(a.decay[tb + t0 + t]) : 1.f;
      sm.eta[t] = in ? to_f32(a.lr[tb + t0 + t]) : 0.f;
      sm.beta[t] = in ? (g.momentum ? to_f32(a.beta[tb + t0 + t]) : 0.f) : 1.f;
    }
    __syncthreads();
    if (tid == 0) {
      float ac = 1.f, kc = 0.f, bc = 1.f;
      for (int t = 0; t < CH; ++t) {
        sm.acoef[t] = ac;
        sm.kcoef[t] = kc;
        bc = sm.beta[t] * bc;
        ac = sm.alpha[t] * ac;
        kc = sm.alpha[t] * kc + sm.eta[t] * bc;
      }
      sm.endc[0] = ac; sm.endc[1] = kc; sm.endc[2] = bc;
    }
    __syncthreads();
    const float a_end = sm.endc[0], k_end = sm.endc[1], b_end = sm.endc[2];
    const bool clamp_in = (c > 0) && clamp_after(g, t0);
#pragma unroll
    for (int j = 0; j < NOWN; ++j) {
      const int kt = wave + kWaves * j;
      if (kt >= NKT) continue;
      const int n0 = kt * 16;
      f32x4 aa = zero4(), ak = zero4();
      for (int k0 = 0; k0 < CH; k0 += M::KS) {
        const typename M::frag fb = frag_ld<T>(&sm.psi[0][0], 1, DK + 8, n0, k0);
        aa = M::mma(frag_ld_kscaled<T>(&sm.dyT[0][0], CH + 1, 1, 0, k0, sm.acoef), fb, aa);
        ak = M::mma(frag_ld_kscaled<T>(&sm.dyT[0][0], CH + 1, 1, 0, k0, sm.kcoef), fb, ak);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 4 * (lane >> 4) + r, k = n0 + (lane & 15);
        const float lam = a_end * dS[j][r] + aa[r];
        const float mu = g.momentum ? (b_end * dZ[j][r] - k_end * dS[j][r] - ak[r]) : 0.f;
        if (c > 0) {
          float m = 1.f;
          if (clamp_in) {
            const size_t so = ((size_t)bh * g.nc + (c - 1)) * cs + (size_t)(row0 + i) * DK + k;
            m = clamp_mask(a.saved[so]);
          }
          dS[j][r] = lam * m;
          dZ[j][r] = mu;
        } else {
          const size_t off = sb + (size_t)(row0 + i) * DK + k;
          a.dS0[off] = lam;
          if (g.momentum && a.dZ0) a.dZ0[off] = mu;
        }
      }
    }
    __syncthreads();
  }
}

// =============================================================================================
// B2: per-chunk gradients
// =============================================================================================
template <typename T, int CH, int DK, int DV>
struct ChunkSmem {
  static constexpr int SPM = CH + kHaloPad;
  // phases 0-3
  union {
    struct {
      T phi[SPM][DK + 8];
      T psi[CH][DK + 8];
      T dy[CH][DV + 8];
      T deltaT[SPM][DV + 8];
      T Q[CH][SPM + 8];
      T Qp[CH][SPM + 8];
      T dD[DV][SPM + 8];
      float wsh[CH][SPM + 1];    // Ws[s, tau-1]
    } m;
    struct {
      float LWs[CH][CH + 1];     // sum_s Lm[q,s] Ws[s,tau]
      float LWz[CH][CH + 1];     // sum_s Lm[q,s] Wz[s,tau]
    } p4;
  } u;
  float Lm[CH][SPM + 1];         // (dy_q.delta_s)(psi_q.phi_s)
  float hS[SPM], hZ[SPM];        // <dS_end, P_s>, <dZ_end, P_s>
  float fS[CH], fZ[CH];          // dy_q^T S_in psi_q, dy_q^T Z_in psi_q
  float HWsS[CH], HWzS[CH], HWzZ[CH];
  float alpha[CH], eta[CH], beta[CH];
  float ug[SPM];
  float wl[CH * kMaxWindow];
  float wsend[SPM], wzend[SPM];
  float A1[CH + 1], K1[CH + 1], B1[CH + 1];   // a, kappa, b at tau' = -1 .. CH-1 (index tau'+1)
  float gram[4];                 // <dS_end,S_in>, <dS_end,Z_in>, <dZ_end,Z_in>
  float red[kWaves][4];
};

template <typename T>
__device__ __forceinline__ float src_weight(int gate_mode, const float* ug, const float* wl, int e, int s, int t, int j) {
  return gate_mode == GATE_TOKEN ? ug[s] : (gate_mode == GATE_LAG ? wl[t * e + j] : 1.f);
}

template <typename T, int CH, int DK, int DV>
__global__ __launch_bounds__(kThreads) void k_bwd_chunk(const Geom g, const BwdPtrs<T> a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  typedef ChunkSmem<T, CH, DK, DV> Sm;
  Sm& sm = *reinterpret_cast<Sm*>(smem_raw);
  constexpr int SPM = Sm::SPM;
  typedef MM<T> M;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int c = blockIdx.x, bh = blockIdx.y;
  const int H = g.H, SP = g.SP, e = g.e;
  const int t0 = c * g.Lc;
  const int t1 = min(g.T, t0 + g.Lc);
  const int L = t1 - t0;
  const bool bufchunk = (c == 0) && g.has_buf;
  const size_t tb = (size_t)bh * g.T;
  const size_t sb = (size_t)bh * DV * DK;
  const size_t cst = (size_t)2 * DV * DK;
  const float* Sref = a.S_ref + sb;
  // chunk-start forward states
  const float* Sin = (c == 0) ? a.S0 + sb : a.saved + ((size_t)bh * g.nc + c - 1) * cst;
  const float* Zin = (c == 0) ? (a.Z0 ? a.Z0 + sb : nullptr) : a.saved + ((size_t)bh * g.nc + c - 1) * cst + (size_t)DV * DK;
  if (!g.momentum) Zin = nullptr;
  const bool clamp_in = (c > 0) && clamp_after(g, t0);
  const float* dSe = a.adj + ((size_t)bh * g.nc + c) * cst;
  const float* dZe = dSe + (size_t)DV * DK;

  // ---------------------------------------------------------------- phase 0: loads
  for (int idx = tid; idx < SP * DK; idx += kThreads) {
    const int s = idx / DK, k = idx % DK;
    const int p = t0 - H + s;
    float val = 0.f;
    if (s < H + L && p >= 0) val = ld_map(a.k, (tb + p) * DK + k, g.map_mode, g.map_deg);
    sm.u.m.phi[s][k] = from_f32<T>(val);
  }
  for (int idx = tid; idx < CH * DK; idx += kThreads) {
    const int t = idx / DK, k = idx % DK;
    float val = 0.f;
    if (t < L) val = ld_map(a.q, (tb + t0 + t) * DK + k, g.map_mode, g.map_deg);
    sm.u.m.psi[t][k] = from_f32<T>(val);
  }
  for (int idx = tid; idx < CH * DV; idx += kThreads) {
    const int t = idx / DV, i = idx % DV;
    sm.u.m.dy[t][i] = from_f32<T>((t < L && a.dy) ? to_f32(a.dy[(tb + t0 + t) * DV + i]) : 0.f);
  }
  if (tid < CH) {
    const int t = tid;
    const bool in = t < L;
    sm.alpha[t] = in ? to_f32(a.decay[tb + t0 + t]) : 1.f;
    sm.eta[t] = in ? to_f32(a.lr[tb + t0 + t]) : 0.f;
    sm.beta[t] = in ? (g.momentum ? to_f32(a.beta[tb + t0 + t]) : 0.f) : 1.f;
    sm.fS[t] = 0.f; sm.fZ[t] = 0.f;
  }
  for (int s = tid; s < SPM; s += kThreads) { sm.hS[s] = 0.f; sm.hZ[s] = 0.f; }
  if (g.gate_mode == GATE_TOKEN) {
    for (int s = tid; s < SP; s += kThreads) {
      const int p = t0 - H + s;
      sm.ug[s] = (s < H + L) ? (p >= 0 ? to_f32(a.gate[tb + p]) : 1.f) : 0.f;
    }
  } else if (g.gate_mode == GATE_LAG) {
    for (int idx = tid; idx < CH * e; idx += kThreads) {
      const int t = idx / e, j = idx % e;
      sm.wl[idx] = (t < L) ? to_f32(a.gate[(tb + t0 + t) * e + j]) : 0.f;
    }
  }
  // Gram scalars over the full state
  {
    float gss = 0.f, gsz = 0.f, gzz = 0.f;
    for (int idx = tid; idx < DV * DK; idx += kThreads) {
      float s_in = Sin[idx];
      if (clamp_in) s_in = clamp100(s_in);
      const float z_in = Zin ? Zin[idx] : 0.f;
      const float ds = dSe[idx], dz = dZe[idx];
      gss += ds * s_in; gsz += ds * z_in; gzz += dz * z_in;
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
      for (int w = 0; w < kWaves; ++w) s += sm.red[w][q];
      sm.gram[q] = s;
    }
  }
  // buffer sources: hS, hZ = <dS_end, B_s>, <dZ_end, B_s>
  if (bufchunk) {
    for (int s = 0; s < H; ++s) {
      const float* Bs = a.buf_in + ((size_t)bh * H + s) * DV * DK;
      float hs = 0.f, hz = 0.f;
      for (int idx = tid; idx < DV * DK; idx += kThreads) { hs += dSe[idx] * Bs[idx]; hz += dZe[idx] * Bs[idx]; }
      for (int off = 32; off > 0; off >>= 1) { hs += __shfl_xor(hs, off); hz += __shfl_xor(hz, off); }
      if (lane == 0) { atomicAdd(&sm.hS[s], hs); atomicAdd(&sm.hZ[s], hz); }
    }
  }
  // coefficient recurrences
  if (tid < SP) {
    const int s = tid;
    float ws = 0.f, wz = 0.f;
    for (int t = 0; t < CH; ++t) {
      sm.u.m.wsh[t][s] = ws;
      const int j = t + H - s;
      const float w = (j >= 0 && j < e && t < L) ? src_weight<T>(g.gate_mode, sm.ug, sm.wl, e, s, t, j) : 0.f;
      wz = sm.beta[t] * wz + w;
      ws = sm.alpha[t] * ws + sm.eta[t] * wz;
    }
    sm.wsend[s] = ws;
    sm.wzend[s] = wz;
  } else if (tid == kThreads - 1) {
    float ac = 1.f, kc = 0.f, bc = 1.f;
    sm.A1[0] = 1.f; sm.K1[0] = 0.f; sm.B1[0] = 1.f;
    for (int t = 0; t < CH; ++t) {
      bc = sm.beta[t] * bc;
      ac = sm.alpha[t] * ac;
      kc = sm.alpha[t] * kc + sm.eta[t] * bc;
      sm.A1[t + 1] = ac; sm.K1[t + 1] = kc; sm.B1[t + 1] = bc;
    }
  }
  __syncthreads();

  // ---------------------------------------------------------------- phase 1
  // G1: delta^T[s, i] = phi_s . S_ref[i, :] - v_s[i]
  {
    const int nti = DV / 16;
    for (int tile = wave; tile < (SP / 16) * nti; tile += kWaves) {
      const int m0 = (tile / nti) * 16, n0 = (tile % nti) * 16;
      f32x4 acc = zero4();
      for (int k0 = 0; k0 < DK; k0 += M::KS)
        acc = M::mma(frag_ld_row<T>(&sm.u.m.phi[0][0], DK + 8, m0, k0), frag_ld<T>(Sref, DK, 1, n0, k0), acc);
      const int i = n0 + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int s = m0 + 4 * (lane >> 4) + r;
        const int p = t0 - H + s;
        float d = 0.f;
        if (s < H + L && p >= 0) d = acc[r] - to_f32(a.v[(tb + p) * DV + i]);
        sm.u.m.deltaT[s][i] = from_f32<T>(d);
      }
    }
  }
  __syncthreads();
  // G2/G3: Kmat = psi phi^T, K3 = dy delta  ->  Q, Q', Lm
  {
    const int nts = SP / 16;
    for (int tile = wave; tile < (CH / 16) * nts; tile += kWaves) {
      const int m0 = (tile / nts) * 16, n0 = (tile % nts) * 16;
      f32x4 kk = zero4(), k3 = zero4();
      for (int k0 = 0; k0 < DK; k0 += M::KS)
        kk = M::mma(frag_ld_row<T>(&sm.u.m.psi[0][0], DK + 8, m0, k0),
                    frag_ld_row<T>(&sm.u.m.phi[0][0], DK + 8, n0, k0), kk);
      for (int k0 = 0; k0 < DV; k0 += M::KS)
        k3 = M::mma(frag_ld_row<T>(&sm.u.m.dy[0][0], DV + 8, m0, k0),
                    frag_ld_row<T>(&sm.u.m.deltaT[0][0], DV + 8, n0, k0), k3);
      const int s = n0 + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = m0 + 4 * (lane >> 4) + r;
        const float w = sm.u.m.wsh[t][s];
        sm.u.m.Q[t][s] = from_f32<T>(w * kk[r]);
        sm.u.m.Qp[t][s] = from_f32<T>(w * k3[r]);
        sm.Lm[t][s] = kk[r] * k3[r];
      }
    }
  }
  __syncthreads();

  // ---------------------------------------------------------------- phase 2
  // G4: dDelta[i, s] = Wz_end[s] (dZ_end phi_s)_i - Ws_end[s] (dS_end phi_s)_i - sum_q dy_q[i] Q[q, s]
  {
    const int nts = SP / 16;
    for (int tile = wave; tile < (DV / 16) * nts; tile += kWaves) {
      const int m0 = (tile / nts) * 16, n0 = (tile % nts) * 16;
      f32x4 az = zero4(), as = zero4(), aq = zero4();
      for (int k0 = 0; k0 < DK; k0 += M::KS) {
        const typename M::frag fb = frag_ld_row<T>(&sm.u.m.phi[0][0], DK + 8, n0, k0);
        as = M::mma(frag_ld<T>(dSe, DK, 1, m0, k0), fb, as);
        az = M::mma(frag_ld<T>(dZe, DK, 1, m0, k0), fb, az);   // dZ_end == 0 without momentum
      }
      for (int k0 = 0; k0 < CH; k0 += M::KS)
        aq = M::mma(frag_ld<T>(&sm.u.m.dy[0][0], 1, DV + 8, m0, k0),
                    frag_ld<T>(&sm.u.m.Q[0][0], 1, SPM + 8, n0, k0), aq);
      const int s = n0 + (lane & 15);
      const float wz = sm.wzend[s], ws = sm.wsend[s];
      float hs = 0.f, hz = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = m0 + 4 * (lane >> 4) + r;
        const float d = to_f32(sm.u.m.deltaT[s][i]);
        hs += d * as[r];
        hz += d * az[r];
        sm.u.m.dD[i][s] = from_f32<T>(wz * az[r] - ws * as[r] - aq[r]);
      }
      // reduce over the 4 lane groups holding other rows of the same column
      hs += __shfl_xor(hs, 16); hs += __shfl_xor(hs, 32);
      hz += __shfl_xor(hz, 16); hz += __shfl_xor(hz, 32);
      if (lane < 16) { atomicAdd(&sm.hS[s], hs); atomicAdd(&sm.hZ[s], hz); }
    }
  }
  __syncthreads();

  // ---------------------------------------------------------------- phase 3
  // dv (= -dDelta) for sources; final for tokens whose window stays in the chunk
  {
    const int tail0 = t1 - H;   // tokens >= tail0 also receive gradient from the next chunk
    for (int idx = tid; idx < (H + L) * DV; idx += kThreads) {
      const int s = idx / DV, i = idx % DV;
      const int p = t0 - H + s;
      if (p < 0) continue;
      const float val = -to_f32(sm.u.m.dD[i][s]);
      if (s < H) {
        if (c > 0) a.halo_part[(((size_t)bh * g.nc + c) * H + s) * (DV + DK) + i] = val;
      } else if (p >= tail0) {
        a.tail_part[(((size_t)bh * g.nc + c) * H + (p - tail0)) * (DV + DK) + i] = val;
      } else {
        a.dv[(tb + p) * DV + i] = from_f32<T>(val);
      }
    }
  }
  // G5: dphi[s, k]
  {
    const int ntk = DK / 16;
    const int tail0 = t1 - H;
    for (int tile = wave; tile < (SP / 16) * ntk; tile += kWaves) {
      const int m0 = (tile / ntk) * 16, n0 = (tile % ntk) * 16;
      f32x4 a1 = zero4(), a2 = zero4(), a3 = zero4(), a4 = zero4();
      for (int k0 = 0; k0 < DV; k0 += M::KS) {
        const typename M::frag fa = frag_ld_row<T>(&sm.u.m.deltaT[0][0], DV + 8, m0, k0);
        a2 = M::mma(fa, frag_ld<T>(dSe, 1, DK, n0, k0), a2);
        a1 = M::mma(fa, frag_ld<T>(dZe, 1, DK, n0, k0), a1);
        a4 = M::mma(frag_ld<T>(&sm.u.m.dD[0][0], 1, SPM + 8, m0, k0), frag_ld<T>(Sref, 1, DK, n0, k0), a4);
      }
      for (int k0 = 0; k0 < CH; k0 += M::KS)
        a3 = M::mma(frag_ld<T>(&sm.u.m.Qp[0][0], 1, SPM + 8, m0, k0),
                    frag_ld<T>(&sm.u.m.psi[0][0], 1, DK + 8, n0, k0), a3);
      const int k = n0 + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int s = m0 + 4 * (lane >> 4) + r;
        const int p = t0 - H + s;
        if (s >= H + L || p < 0) continue;
        const float val = sm.wzend[s] * a1[r] - sm.wsend[s] * a2[r] - a3[r] + a4[r];
        if (s < H) {
          if (c > 0) a.halo_part[(((size_t)bh * g.nc + c) * H + s) * (DV + DK) + DV + k] = val;
        } else if (p >= tail0) {
          a.tail_part[(((size_t)bh * g.nc + c) * H + (p - tail0)) * (DV + DK) + DV + k] = val;
        } else {
          float outv = val;
          if (g.map_mode == MAP_ELEMENTWISE) outv *= poly_map_grad(to_f32(a.k[(tb + p) * DK + k]), g.map_deg);
          a.dk[(tb + p) * DK + k] = from_f32<T>(outv);
        }
      }
    }
  }
  // G6: dS_ref partial[i, k] = sum_s dDelta[i, s] phi_s[k]
  {
    const int ntk = DK / 16;
    float* dst = a.dsref_part + ((size_t)bh * g.nc + c) * DV * DK;
    for (int tile = wave; tile < (DV / 16) * ntk; tile += kWaves) {
      const int m0 = (tile / ntk) * 16, n0 = (tile % ntk) * 16;
      f32x4 acc = zero4();
      for (int k0 = 0; k0 < SP; k0 += M::KS)
        acc = M::mma(frag_ld_row<T>(&sm.u.m.dD[0][0], SPM + 8, m0, k0),
                     frag_ld<T>(&sm.u.m.phi[0][0], 1, DK + 8, n0, k0), acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = m0 + 4 * (lane >> 4) + r, k = n0 + (lane & 15);
        dst[(size_t)i * DK + k] = acc[r];
      }
    }
  }
  // G7: dpsi[t, k] = a_{t-1} (dy_t S_in)_k - kappa_{t-1} (dy_t Z_in)_k - sum_s Q'[t, s] phi_s[k]
  {
    const int ntk = DK / 16;
    for (int tile = wave; tile < (CH / 16) * ntk; tile += kWaves) {
      const int m0 = (tile / ntk) * 16, n0 = (tile % ntk) * 16;
      f32x4 as = zero4(), az = zero4(), aq = zero4();
      for (int k0 = 0; k0 < DV; k0 += M::KS) {
        const typename M::frag fa = frag_ld_row<T>(&sm.u.m.dy[0][0], DV + 8, m0, k0);
        // Bt element (k, i) = S_in[i][k]
        typename M::frag fs;
        if (clamp_in) {
          const int l = lane;
          const int kb = k0 + (l >> 4) * M::KL;
          const float* q = Sin + (size_t)kb * DK + n0 + (l & 15);
          if constexpr (M::KL == 1) fs = static_cast<T>(clamp100(q[0]));
          else {
#pragma unroll
            for (int ee = 0; ee < M::KL; ++ee) fs[ee] = static_cast<T>(clamp100(q[(size_t)ee * DK]));
          }
        } else {
          fs = frag_ld<T>(Sin, 1, DK, n0, k0);
        }
        as = M::mma(fa, fs, as);
        az = M::mma(fa, frag_ld_or_zero<T>(Zin, 1, DK, n0, k0), az);
      }
      for (int k0 = 0; k0 < SP; k0 += M::KS)
        aq = M::mma(frag_ld_row<T>(&sm.u.m.Qp[0][0], SPM + 8, m0, k0),
                    frag_ld<T>(&sm.u.m.phi[0][0], 1, DK + 8, n0, k0), aq);
      const int k = n0 + (lane & 15);
      f32x4 dpsi;
      float fs_part[4], fz_part[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = m0 + 4 * (lane >> 4) + r;
        dpsi[r] = sm.A1[t] * as[r] - sm.K1[t] * az[r] - aq[r];
        const float ps = to_f32(sm.u.m.psi[t][k]);
        fs_part[r] = as[r] * ps;
        fz_part[r] = az[r] * ps;
      }
      if (bufchunk) {
        // dense buffer sources: dpsi_t -= Ws[s,t-1] B_s^T dy_t ;  Lm[t, s] = dy_t^T B_s psi_t
        for (int s = 0; s < H; ++s) {
          const float* Bs = a.buf_in + ((size_t)bh * H + s) * DV * DK;
          f32x4 ab = zero4();
          for (int k0 = 0; k0 < DV; k0 += M::KS)
            ab = M::mma(frag_ld_row<T>(&sm.u.m.dy[0][0], DV + 8, m0, k0), frag_ld<T>(Bs, 1, DK, n0, k0), ab);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = m0 + 4 * (lane >> 4) + r;
            dpsi[r] -= sm.u.m.wsh[t][s] * ab[r];
            float lm = ab[r] * to_f32(sm.u.m.psi[t][k]);
            for (int off = 8; off > 0; off >>= 1) lm += __shfl_xor(lm, off);
            if ((lane & 15) == 0) atomicAdd(&sm.Lm[t][s], lm);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = m0 + 4 * (lane >> 4) + r;
        // reduce fS/fZ over the 16 lanes of this row group (k columns), then across tiles
        float fsv = fs_part[r], fzv = fz_part[r];
        for (int off = 8; off > 0; off >>= 1) { fsv += __shfl_xor(fsv, off); fzv += __shfl_xor(fzv, off); }
        if ((lane & 15) == 0) { atomicAdd(&sm.fS[t], fsv); atomicAdd(&sm.fZ[t], fzv); }
        if (t < L) {
          float outv = dpsi[r];
          if (g.map_mode == MAP_ELEMENTWISE) outv *= poly_map_grad(to_f32(a.q[(tb + t0 + t) * DK + k]), g.map_deg);
          a.dq[(tb + t0 + t) * DK + k] = from_f32<T>(outv);
        }
      }
    }
  }
  // d buffer_in[s] = Wz_end[s] dZ_end - Ws_end[s] dS_end - sum_q Ws[s, q-1] dy_q psi_q^T   (chunk 0)
  if (bufchunk) {
    const int ntk = DK / 16;
    for (int s = 0; s < H; ++s) {
      float* dst = a.dbuf_in + ((size_t)bh * H + s) * DV * DK;
      for (int tile = wave; tile < (DV / 16) * ntk; tile += kWaves) {
        const int m0 = (tile / ntk) * 16, n0 = (tile % ntk) * 16;
        f32x4 acc = zero4();
        for (int k0 = 0; k0 < CH; k0 += M::KS) {
          // A element (i, q) = dy[q][i] * Ws[s, q-1]
          typename M::frag fa;
          const int l = lane;
          const int qb = k0 + (l >> 4) * M::KL;
          const int i = m0 + (l & 15);
          if constexpr (M::KL == 1) fa = static_cast<T>(to_f32(sm.u.m.dy[qb][i]) * sm.u.m.wsh[qb][s]);
          else {
#pragma unroll
            for (int ee = 0; ee < M::KL; ++ee)
              fa[ee] = static_cast<T>(to_f32(sm.u.m.dy[qb + ee][i]) * sm.u.m.wsh[qb + ee][s]);
          }
          acc = M::mma(fa, frag_ld<T>(&sm.u.m.psi[0][0], 1, DK + 8, n0, k0), acc);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = m0 + 4 * (lane >> 4) + r, k = n0 + (lane & 15);
          const size_t o = (size_t)i * DK + k;
          const float dz = g.momentum ? dZe[o] : 0.f;
          dst[o] = sm.wzend[s] * dz - sm.wsend[s] * dSe[o] - acc[r];
        }
      }
    }
  }
  __syncthreads();

  // ---------------------------------------------------------------- phase 4: scalar gradients
  // Recurrences over tau' for the window-weighted Gram terms (sources -> targets):
  //   LWz[q,t] = beta_t LWz[q,t-1] + sum_j w(t,j) Lm[q, s(t,j)],  LWs[q,t] = alpha_t LWs[q,t-1] + eta_t LWz[q,t]
  // and the same for hS, hZ (HW*).   (u.m is dead from here on; u.p4 reuses it.)
  if (tid < CH) {
    const int q = tid;
    float lz = 0.f, ls = 0.f;
    for (int t = 0; t < CH; ++t) {
      float acc = 0.f;
      for (int j = 0; j < e && t < L; ++j) {
        const int s = t + H - j;
        acc += src_weight<T>(g.gate_mode, sm.ug, sm.wl, e, s, t, j) * sm.Lm[q][s];
      }
      lz = sm.beta[t] * lz + acc;
      ls = sm.alpha[t] * ls + sm.eta[t] * lz;
      sm.u.p4.LWs[q][t] = ls;
      sm.u.p4.LWz[q][t] = lz;
    }
  } else if (tid == CH) {
    float hzs = 0.f, hss = 0.f, hzz = 0.f;
    for (int t = 0; t < CH; ++t) {
      float as = 0.f, az = 0.f;
      for (int j = 0; j < e && t < L; ++j) {
        const int s = t + H - j;
        const float w = src_weight<T>(g.gate_mode, sm.ug, sm.wl, e, s, t, j);
        as += w * sm.hS[s];
        az += w * sm.hZ[s];
      }
      hzs = sm.beta[t] * hzs + as;
      hss = sm.alpha[t] * hss + sm.eta[t] * hzs;
      hzz = sm.beta[t] * hzz + az;
      sm.HWsS[t] = hss; sm.HWzS[t] = hzs; sm.HWzZ[t] = hzz;
    }
  }
  __syncthreads();
  if (tid < L) {
    const int t = tid;
    const float gss = sm.gram[0], gsz = sm.gram[1], gzz = sm.gram[2];
    // values at tau' = t - 1 (index t in the shifted arrays) and at tau' = t (index t + 1)
    const float am1 = sm.A1[t], km1 = sm.K1[t], bm1 = sm.B1[t];
    const float b0 = sm.B1[t + 1];
    const float HWsS_m1 = t > 0 ? sm.HWsS[t - 1] : 0.f;
    const float HWzS_m1 = t > 0 ? sm.HWzS[t - 1] : 0.f;
    const float HWzZ_m1 = t > 0 ? sm.HWzZ[t - 1] : 0.f;
    const float ES_m1 = am1 * gss - km1 * gsz - HWsS_m1;
    const float EZS_m1 = bm1 * gsz + HWzS_m1;
    const float EZZ_m1 = bm1 * gzz + HWzZ_m1;
    const float EZS_0 = b0 * gsz + sm.HWzS[t];
    float da = 0.f, de = 0.f, db = 0.f;
    float dwj[kMaxWindow];
    for (int j = 0; j < e; ++j) dwj[j] = 0.f;
    float Ar = 1.f, Br = 1.f, Mr = sm.eta[t];
    for (int q = t + 1; q < L; ++q) {
      const float LWs_m1 = t > 0 ? sm.u.p4.LWs[q][t - 1] : 0.f;
      const float LWz_m1 = t > 0 ? sm.u.p4.LWz[q][t - 1] : 0.f;
      const float FS_m1 = am1 * sm.fS[q] - km1 * sm.fZ[q] - LWs_m1;
      const float FZ_0 = b0 * sm.fZ[q] + sm.u.p4.LWz[q][t];
      const float FZ_m1 = bm1 * sm.fZ[q] + LWz_m1;
      da += Ar * FS_m1;
      de += Ar * FZ_0;
      db += Mr * FZ_m1;
      for (int j = 0; j < e; ++j) dwj[j] += Mr * sm.Lm[q][t + H - j];
      Ar *= sm.alpha[q];
      Br *= sm.beta[q];
      Mr = sm.alpha[q] * Mr + sm.eta[q] * Br;
    }
    da += Ar * ES_m1;
    de = -(de + Ar * EZS_0);
    db = Br * EZZ_m1 - Mr * EZS_m1 - db;
    const size_t tt = tb + t0 + t;
    a.ddecay[tt] = from_f32<T>(da);
    a.dlr[tt] = from_f32<T>(de);
    if (g.momentum && a.dbeta) a.dbeta[tt] = from_f32<T>(db);
    if (g.gate_mode != GATE_NONE) {
      for (int j = 0; j < e; ++j) {
        const int s = t + H - j;
        const float v = Br * sm.hZ[s] - Mr * sm.hS[s] - dwj[j];
        if (g.gate_mode == GATE_LAG) a.dgate[tt * e + j] = from_f32<T>(v);
        else a.dw[tt * e + j] = v;
      }
    }
  }
}

// =============================================================================================
// B3: chunk-boundary fixup, d buffer_out terms, token-gate reduction, feature-map derivative.
// grid (nc, BH)
// =============================================================================================
template <typename T, int DK, int DV>
__global__ __launch_bounds__(kThreads) void k_bwd_fixup(const Geom g, const BwdPtrs<T> a) {
  __shared__ float sphi[DK], sdel[DV], sdd[DV], sdb[DV];
  const int c = blockIdx.x, bh = blockIdx.y;
  const int H = g.H, e = g.e;
  const int t0 = c * g.Lc, t1 = min(g.T, t0 + g.Lc);
  const size_t tb = (size_t)bh * g.T;
  const int tid = threadIdx.x;
  // token-gate gradient du_p = sum_j dw[p + j, j]  (+ d buffer_out term below)
  if (g.gate_mode == GATE_TOKEN) {
    for (int p = t0 + tid; p < t1; p += kThreads) {
      if (p >= g.T - H && a.dbuf_out) continue;   // finished in the tail loop
      float du = 0.f;
      for (int j = 0; j < e && p + j < g.T; ++j) du += a.dw[(tb + p + j) * e + j];
      a.dgate[tb + p] = from_f32<T>(du);
    }
  }
  if (H == 0) return;
  const int tail0 = t1 - H;
  for (int h = 0; h < H; ++h) {
    const int p = tail0 + h;
    if (p < t0 || p < 0) continue;       // belongs to the previous chunk (short last chunk)
    const size_t tp = (((size_t)bh * g.nc + c) * H + h) * (DV + DK);
    const bool has_next = c + 1 < g.nc;
    const size_t hp = has_next ? (((size_t)bh * g.nc + c + 1) * H + h) * (DV + DK) : 0;
    const bool outbuf = (a.dbuf_out != nullptr) && (p >= g.T - H);
    const int kb = p - (g.T - H);
    __syncthreads();
    if (outbuf) {
      // Gamma_p += c_p dBufOut[kb]: ddelta_x = c_p dBuf phi_p ; dphi_x = c_p dBuf^T delta_p + S_ref^T ddelta_x
      for (int k = tid; k < DK; k += kThreads) sphi[k] = ld_map(a.k, (tb + p) * DK + k, g.map_mode, g.map_deg);
      __syncthreads();
      const float cp = (g.gate_mode == GATE_TOKEN) ? to_f32(a.gate[tb + p]) : 1.f;
      const float* dB = a.dbuf_out + ((size_t)bh * H + kb) * DV * DK;
      const float* Sr = a.S_ref + (size_t)bh * DV * DK;
      for (int i = tid; i < DV; i += kThreads) {
        float acc = 0.f, accd = 0.f;
        for (int k = 0; k < DK; ++k) { acc += Sr[(size_t)i * DK + k] * sphi[k]; accd += dB[(size_t)i * DK + k] * sphi[k]; }
        sdel[i] = acc - to_f32(a.v[(tb + p) * DV + i]);
        sdb[i] = accd;
        sdd[i] = cp * accd;
      }
      __syncthreads();
      if (tid == 0 && g.gate_mode == GATE_TOKEN) {
        // du_p = sum_j dw[p + j, j] + <dBuf, delta_p phi_p^T>
        float du = 0.f;
        for (int i = 0; i < DV; ++i) du += sdel[i] * sdb[i];
        for (int j = 0; j < e && p + j < g.T; ++j) du += a.dw[(tb + p + j) * e + j];
        a.dgate[tb + p] = from_f32<T>(du);
      }
      // dS_ref += ddelta_x phi_p^T  (this chunk's partial slot; only this block writes it)
      float* dsr = a.dsref_part + ((size_t)bh * g.nc + c) * DV * DK;
      for (int idx = tid; idx < DV * DK; idx += kThreads) dsr[idx] += sdd[idx / DK] * sphi[idx % DK];
    }
    for (int i = tid; i < DV; i += kThreads) {
      float val = a.tail_part[tp + i] + (has_next ? a.halo_part[hp + i] : 0.f);
      if (outbuf) val -= sdd[i];
      a.dv[(tb + p) * DV + i] = from_f32<T>(val);
    }
    for (int k = tid; k < DK; k += kThreads) {
      float val = a.tail_part[tp + DV + k] + (has_next ? a.halo_part[hp + DV + k] : 0.f);
      if (outbuf) {
        const float cp = (g.gate_mode == GATE_TOKEN) ? to_f32(a.gate[tb + p]) : 1.f;
        const float* dB = a.dbuf_out + ((size_t)bh * H + kb) * DV * DK;
        const float* Sr = a.S_ref + (size_t)bh * DV * DK;
        float acc = 0.f;
        for (int i = 0; i < DV; ++i) acc += cp * dB[(size_t)i * DK + k] * sdel[i] + Sr[(size_t)i * DK + k] * sdd[i];
        val += acc;
      }
      if (g.map_mode == MAP_ELEMENTWISE) val *= poly_map_grad(to_f32(a.k[(tb + p) * DK + k]), g.map_deg);
      a.dk[(tb + p) * DK + k] = from_f32<T>(val);
    }
  }
  // buffer pass-through when T < e - 1: buffer_out[k'] = buffer_in[T + k']
  if (c == 0 && a.dbuf_out && a.dbuf_in && g.T < H) {
    __syncthreads();
    for (int kq = 0; kq + g.T < H; ++kq) {
      const float* src = a.dbuf_out + ((size_t)bh * H + kq) * DV * DK;
      float* dst = a.dbuf_in + ((size_t)bh * H + g.T + kq) * DV * DK;
      for (int idx = tid; idx < DV * DK; idx += kThreads) dst[idx] += src[idx];
    }
  }
}

// B4: dS_ref = sum over chunks of the partials.   grid (DV*DK/256, BH)
__global__ __launch_bounds__(kThreads) void k_reduce_dsref(const Geom g, const float* part, float* out) {
  const int bh = blockIdx.y;
  const int idx = blockIdx.x * kThreads + threadIdx.x;
  const int n = g.DV * g.DK;
  if (idx >= n) return;
  float acc = 0.f;
  for (int c = 0; c < g.nc; ++c) acc += part[((size_t)bh * g.nc + c) * n + idx];
  out[(size_t)bh * n + idx] = acc;
}

template <typename T, int CH, int DK, int DV>
hipError_t launch_bwd(const Geom& g, const BwdPtrs<T>& a, hipStream_t stream) {
  hipError_t err;
  {
    const size_t smem = sizeof(AdjSmem<T, CH, DK>);
    err = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_bwd_adjoint_walk<T, CH, DK, DV>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (err != hipSuccess) return err;
    prof_begin(KID_BWD_ADJOINT, stream);
    hipLaunchKernelGGL((k_bwd_adjoint_walk<T, CH, DK, DV>), dim3(DV / 16, g.BH), dim3(kThreads), smem, stream, g, a);
    prof_end(KID_BWD_ADJOINT, stream);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  {
    const size_t smem = sizeof(ChunkSmem<T, CH, DK, DV>);
    err = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_bwd_chunk<T, CH, DK, DV>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (err != hipSuccess) return err;
    prof_begin(KID_BWD_CHUNK, stream);
    hipLaunchKernelGGL((k_bwd_chunk<T, CH, DK, DV>), dim3(g.nc, g.BH), dim3(kThreads), smem, stream, g, a);
    prof_end(KID_BWD_CHUNK, stream);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  prof_begin(KID_BWD_FIXUP, stream);
  hipLaunchKernelGGL((k_bwd_fixup<T, DK, DV>), dim3(g.nc, g.BH), dim3(kThreads), 0, stream, g, a);
  prof_end(KID_BWD_FIXUP, stream);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  prof_begin(KID_REDUCE_DSREF, stream);
  hipLaunchKernelGGL(k_reduce_dsref, dim3((DV * DK + kThreads - 1) / kThreads, g.BH), dim3(kThreads), 0, stream,
                     g, (const float*)a.dsref_part, a.dS_ref);
  prof_end(KID_REDUCE_DSREF, stream);
  return hipGetLastError();
}

template <typename T, int CH, int DK, int DV>
size_t bwd_smem_bytes() { return sizeof(ChunkSmem<T, CH, DK, DV>); }

#define ATLAS_INST_BWD(T, CH, DK, DV) \
  template hipError_t launch_bwd<T, CH, DK, DV>(const Geom&, const BwdPtrs<T>&, hipStream_t); \
  template size_t bwd_smem_bytes<T, CH, DK, DV>();

ATLAS_INST_BWD(bf16, 64, 64, 64)
ATLAS_INST_BWD(float, 32, 64, 64)
ATLAS_INST_BWD(bf16, 64, 32, 32)
ATLAS_INST_BWD(float, 32, 32, 32)

}  // namespace atlas
