// mem_fwd.hip - forward pass of the chunked memory recurrence (gfx950).
//
// One workgroup owns 16 rows of S (and Z) of one head-batch row bh and walks the sequence
// chunk by chunk (chunk length Lc <= CH). Inside a chunk everything is written in closed form
// over the chunk's sources (its own tokens plus the e-1 previous ones, the "halo"):
//
//   S_tau = a_tau S_in - kappa_tau Z_in - sum_s Ws[s,tau] delta_s phi_s^T
//   Z_tau = b_tau Z_in                  + sum_s Wz[s,tau] delta_s phi_s^T
//   y_tau = S_{tau-1} psi_tau
//
// where the scalar coefficients follow the recurrence itself applied to unit inputs:
//   Wz[s,tau] = beta_tau Wz[s,tau-1] + w(s,tau),   Ws[s,tau] = alpha_tau Ws[s,tau-1] + eta_tau Wz[s,tau]
//   b_tau = beta_tau b_{tau-1}, a_tau = alpha_tau a_{tau-1}, kappa_tau = alpha_tau kappa_{tau-1} + eta_tau b_tau
// The products run on the matrix cores:
//   G1  delta^T[s,i] = phi_s . S_ref[i,:] - v_s[i]
//   G2  Q[tau,s]     = Ws[s,tau-1] * (psi_tau . phi_s)
//   G3  y^T[tau,i]   = -Q delta^T + a_{tau-1} psi S_in^T - kappa_{tau-1} psi Z_in^T
//   G4  U = -delta diag(Ws_end) Phi,  V = delta diag(Wz_end) Phi
//   S_out = a_end S_in - kappa_end Z_in + U,  Z_out = b_end Z_in + V
// The raw chunk-end states are saved for the backward pass; S is clamped at scan_chunk_len
// boundaries (atlas_pytorch/rnn_memory.py:584-601) and at the end (rnn_memory.py:701).
#include "mem_common.h"
#include "mem_params.h"

namespace atlas {

template <typename T, int CH, int DK>
struct FwdSmem {
  static constexpr int SPM = CH + kHaloPad;
  T phi[SPM][DK + 8];
  T psi[CH][DK + 8];
  T Q[CH][SPM + 8];
  float sref[16][DK + 1];
  float S[16][DK + 1];
  float Z[16][DK + 1];
  float delta[16][SPM + 1];
  float wsh[CH][SPM + 1];   // Ws[s, tau-1]
  float alpha[CH], eta[CH], beta[CH];
  float ug[SPM];            // token-mode gate of each source
  float wl[CH * kMaxWindow];// lag-mode weights [tau][j]
  float wsend[SPM], wzend[SPM];
  float acoef[CH], kcoef[CH];  // a_{tau-1}, kappa_{tau-1}
  float endc[4];               // a_end, kappa_end, b_end
};

template <typename T>
__device__ __forceinline__ float ld_map(const T* p, size_t idx, int map_mode, int deg) {
  float x = to_f32(p[idx]);
  return map_mode == MAP_ELEMENTWISE ? poly_map(x, deg) : x;
}

template <typename T, int CH, int DK, int DV>
__global__ __launch_bounds__(kThreads) void k_fwd_walk(const Geom g, const FwdPtrs<T> a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  typedef FwdSmem<T, CH, DK> Sm;
  Sm& sm = *reinterpret_cast<Sm*>(smem_raw);
  constexpr int SPM = Sm::SPM;
  constexpr int NKT = DK / 16;              // k tiles of a 16-row state slab
  constexpr int NOWN = (NKT + kWaves - 1) / kWaves;
  typedef MM<T> M;

  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int row0 = blockIdx.x * 16;
  const int bh = blockIdx.y;
  const int H = g.H, SP = g.SP, e = g.e;
  const size_t tb = (size_t)bh * g.T;       // token base
  const size_t sb = (size_t)bh * DV * DK;   // state base

  for (int idx = tid; idx < 16 * DK; idx += kThreads) {
    const int i = idx / DK, k = idx % DK;
    const size_t off = sb + (size_t)(row0 + i) * DK + k;
    sm.sref[i][k] = a.S_ref[off];
  }
  float Sr[NOWN][4], Zr[NOWN][4];
#pragma unroll
  for (int j = 0; j < NOWN; ++j) {
    const int kt = wave + kWaves * j;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      Sr[j][r] = 0.f; Zr[j][r] = 0.f;
      if (kt < NKT) {
        const int i = 4 * (lane >> 4) + r, k = kt * 16 + (lane & 15);
        const size_t off = sb + (size_t)(row0 + i) * DK + k;
        Sr[j][r] = a.S0[off];
        Zr[j][r] = (g.momentum && a.Z0) ? a.Z0[off] : 0.f;
        sm.S[i][k] = Sr[j][r];
        sm.Z[i][k] = Zr[j][r];
      }
    }
  }

  for (int c = 0; c < g.nc; ++c) {
    const int t0 = c * g.Lc;
    const int t1 = min(g.T, t0 + g.Lc);
    const int L = t1 - t0;
    const bool bufchunk = (c == 0) && g.has_buf;

    // ---- loads: sources (halo + chunk), queries, scalars
    for (int idx = tid; idx < SP * DK; idx += kThreads) {
      const int s = idx / DK, k = idx % DK;
      const int p = t0 - H + s;
      float val = 0.f;
      if (s < H + L && p >= 0) val = ld_map(a.k, (tb + p) * DK + k, g.map_mode, g.map_deg);
      sm.phi[s][k] = from_f32<T>(val);
    }
    for (int idx = tid; idx < CH * DK; idx += kThreads) {
      const int t = idx / DK, k = idx % DK;
      float val = 0.f;
      if (t < L) val = ld_map(a.q, (tb + t0 + t) * DK + k, g.map_mode, g.map_deg);
      sm.psi[t][k] = from_f32<T>(val);
    }
    if (tid < CH) {
      const int t = tid;
      const bool in = t < L;
      sm.alpha[t] = in ? to_f32(a.decay[tb + t0 + t]) : 1.f;
      sm.eta[t] = in ? to_f32(a.lr[tb + t0 + t]) : 0.f;
      sm.beta[t] = in ? (g.momentum ? to_f32(a.beta[tb + t0 + t]) : 0.f) : 1.f;
    }
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
    __syncthreads();

    // ---- G1: delta^T[s, i] = phi_s . S_ref[i, :] - v_s[i]   (M = SP sources, N = 16 rows)
    for (int tile = wave; tile < SP / 16; tile += kWaves) {
      const int m0 = tile * 16;
      f32x4 acc = zero4();
      for (int k0 = 0; k0 < DK; k0 += M::KS)
        acc = M::mma(frag_ld_row<T>(&sm.phi[0][0], DK + 8, m0, k0),
                     frag_ld<T>(&sm.sref[0][0], DK + 1, 1, 0, k0), acc);
      const int i = lane & 15;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int s = m0 + 4 * (lane >> 4) + r;
        const int p = t0 - H + s;
        float d = 0.f;
        if (s < H + L && p >= 0) d = acc[r] - to_f32(a.v[(tb + p) * DV + row0 + i]);
        sm.delta[i][s] = d;
      }
    }

    // ---- coefficients: per source s (threads s < SP) and the state coefficients (last thread)
    if (tid < SP) {
      const int s = tid;
      float ws = 0.f, wz = 0.f;
      for (int t = 0; t < CH; ++t) {
        sm.wsh[t][s] = ws;
        const int j = t + H - s;
        float w = 0.f;
        if (j >= 0 && j < e && t < L) {
          w = (g.gate_mode == GATE_TOKEN) ? sm.ug[s] : (g.gate_mode == GATE_LAG ? sm.wl[t * e + j] : 1.f);
        }
        wz = sm.beta[t] * wz + w;
        ws = sm.alpha[t] * ws + sm.eta[t] * wz;
      }
      sm.wsend[s] = ws;
      sm.wzend[s] = wz;
    } else if (tid == kThreads - 1) {
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

    // ---- G2: Q[tau, s] = Ws[s, tau-1] * (psi_tau . phi_s)
    {
      const int nts = SP / 16;
      for (int tile = wave; tile < (CH / 16) * nts; tile += kWaves) {
        const int m0 = (tile / nts) * 16, n0 = (tile % nts) * 16;
        f32x4 acc = zero4();
        for (int k0 = 0; k0 < DK; k0 += M::KS)
          acc = M::mma(frag_ld_row<T>(&sm.psi[0][0], DK + 8, m0, k0),
                       frag_ld_row<T>(&sm.phi[0][0], DK + 8, n0, k0), acc);
        const int s = n0 + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = m0 + 4 * (lane >> 4) + r;
          sm.Q[t][s] = from_f32<T>(acc[r] * sm.wsh[t][s]);
        }
      }
    }
    __syncthreads();

    // ---- G3: y^T[tau, i]
    for (int tile = wave; tile < CH / 16; tile += kWaves) {
      const int m0 = tile * 16;
      f32x4 aq = zero4(), as = zero4(), az = zero4();
      for (int k0 = 0; k0 < SP; k0 += M::KS)
        aq = M::mma(frag_ld_row<T>(&sm.Q[0][0], SPM + 8, m0, k0),
                    frag_ld<T>(&sm.delta[0][0], SPM + 1, 1, 0, k0), aq);
      for (int k0 = 0; k0 < DK; k0 += M::KS) {
        const typename M::frag fa = frag_ld_row<T>(&sm.psi[0][0], DK + 8, m0, k0);
        as = M::mma(fa, frag_ld<T>(&sm.S[0][0], DK + 1, 1, 0, k0), as);
        az = M::mma(fa, frag_ld<T>(&sm.Z[0][0], DK + 1, 1, 0, k0), az);   // sm.Z == 0 without momentum
      }
      f32x4 yv;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = m0 + 4 * (lane >> 4) + r;
        yv[r] = -aq[r] + sm.acoef[t] * as[r] - sm.kcoef[t] * az[r];
      }
      if (bufchunk) {
        // dense buffer sources s < H: y_tau -= Ws[s, tau-1] * B_s psi_tau
        for (int s = 0; s < H; ++s) {
          const float* Bs = a.buf_in + ((size_t)bh * H + s) * DV * DK + (size_t)row0 * DK;
          f32x4 ab = zero4();
          for (int k0 = 0; k0 < DK; k0 += M::KS)
            ab = M::mma(frag_ld_row<T>(&sm.psi[0][0], DK + 8, m0, k0), frag_ld<T>(Bs, DK, 1, 0, k0), ab);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = m0 + 4 * (lane >> 4) + r;
            yv[r] -= sm.wsh[t][s] * ab[r];
          }
        }
      }
      const int i = lane & 15;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = m0 + 4 * (lane >> 4) + r;
        if (t < L) a.y[(tb + t0 + t) * DV + row0 + i] = from_f32<T>(yv[r]);
      }
    }

    // ---- G4 + state update on the wave's own k tiles
    const float a_end = sm.endc[0], k_end = sm.endc[1], b_end = sm.endc[2];
    const bool do_clamp = clamp_after(g, t1);
#pragma unroll
    for (int j = 0; j < NOWN; ++j) {
      const int kt = wave + kWaves * j;
      if (kt >= NKT) continue;
      const int n0 = kt * 16;
      f32x4 au = zero4(), av = zero4();
      for (int k0 = 0; k0 < SP; k0 += M::KS) {
        const typename M::frag fb = frag_ld<T>(&sm.phi[0][0], 1, DK + 8, n0, k0);
        au = M::mma(frag_ld_kscaled<T>(&sm.delta[0][0], SPM + 1, 1, 0, k0, sm.wsend), fb, au);
        av = M::mma(frag_ld_kscaled<T>(&sm.delta[0][0], SPM + 1, 1, 0, k0, sm.wzend), fb, av);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 4 * (lane >> 4) + r, k = n0 + (lane & 15);
        float U = -au[r], V = av[r];
        if (bufchunk) {
          for (int s = 0; s < H; ++s) {
            const float b = a.buf_in[(((size_t)bh * H + s) * DV + row0 + i) * DK + k];
            U -= sm.wsend[s] * b;
            V += sm.wzend[s] * b;
          }
        }
        const float Sn = a_end * Sr[j][r] - k_end * Zr[j][r] + U;
        const float Zn = g.momentum ? (b_end * Zr[j][r] + V) : 0.f;
        if (a.saved) {
          const size_t so = ((size_t)bh * g.nc + c) * 2 * DV * DK + (size_t)(row0 + i) * DK + k;
          a.saved[so] = Sn;
          a.saved[so + (size_t)DV * DK] = Zn;
        }
        Sr[j][r] = do_clamp ? clamp100(Sn) : Sn;
        Zr[j][r] = Zn;
      }
    }
    __syncthreads();   // every wave finished reading sm.S / sm.Z / phi / psi / delta
#pragma unroll
    for (int j = 0; j < NOWN; ++j) {
      const int kt = wave + kWaves * j;
      if (kt >= NKT) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 4 * (lane >> 4) + r, k = kt * 16 + (lane & 15);
        sm.S[i][k] = Sr[j][r];
        sm.Z[i][k] = Zr[j][r];
      }
    }
  }

  // ---- final states
#pragma unroll
  for (int j = 0; j < NOWN; ++j) {
    const int kt = wave + kWaves * j;
    if (kt >= NKT) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 4 * (lane >> 4) + r, k = kt * 16 + (lane & 15);
      const size_t off = sb + (size_t)(row0 + i) * DK + k;
      a.S_T[off] = g.clamp_final ? clamp100(Sr[j][r]) : Sr[j][r];
      if (g.momentum) a.Z_T[off] = Zr[j][r];
    }
  }
}

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

template <typename T, int CH, int DK, int DV>
hipError_t launch_fwd(const Geom& g, const FwdPtrs<T>& a, hipStream_t stream) {
  const size_t smem = sizeof(FwdSmem<T, CH, DK>);
  hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_fwd_walk<T, CH, DK, DV>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (err != hipSuccess) return err;
  prof_begin(KID_FWD_WALK, stream);
  hipLaunchKernelGGL((k_fwd_walk<T, CH, DK, DV>), dim3(DV / 16, g.BH), dim3(kThreads), smem, stream, g, a);
  prof_end(KID_FWD_WALK, stream);
  err = hipGetLastError();
  if (err != hipSuccess) return err;
  if (g.H > 0 && a.buf_out) {
    prof_begin(KID_BUFFER_OUT, stream);
    hipLaunchKernelGGL((k_buffer_out<T, DK, DV>), dim3(g.H, g.BH), dim3(kThreads), 0, stream, g, a);
    prof_end(KID_BUFFER_OUT, stream);
    err = hipGetLastError();
  }
  return err;
}

template <typename T, int CH, int DK>
size_t fwd_smem_bytes() { return sizeof(FwdSmem<T, CH, DK>); }

#define ATLAS_INST_FWD(T, CH, DK, DV) \
  template hipError_t launch_fwd<T, CH, DK, DV>(const Geom&, const FwdPtrs<T>&, hipStream_t); \
  template size_t fwd_smem_bytes<T, CH, DK>();

ATLAS_INST_FWD(bf16, 64, 64, 64)
ATLAS_INST_FWD(float, 32, 64, 64)
ATLAS_INST_FWD(bf16, 64, 32, 32)
ATLAS_INST_FWD(float, 32, 32, 32)

}  // namespace atlas
