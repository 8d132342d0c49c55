// bwd_scalar.hip - gradients of the per-token scalars (decay alpha, lr eta, momentum beta, window
// gates) of the chunked backward, one workgroup per backward chunk.
//
// Every scalar gradient is a sum over the chunk of decay-weighted inner products between the
// adjoint and the state. The reverse walk (k_bwd_seg) leaves those inner products per chunk in
// a ScalarBlock (Lm, hS, hZ, fS, fZ and the three Grams of the chunk-end adjoint with the
// chunk-start state); this kernel forms the chunk's decay tables and contracts them:
//   F1  Lw[q][t]  = sum_j w(t, j) X_q[t + H - j]        X_q = Lm[q] (q < CH), hS, hZ
//   F2  LWz = Lw B^T-table, LWs = Lw C^T-table           (fp32 matrix cores)
//   F3  one wave per term (dalpha, deta, dbeta, dw[., j]): sums over q of table rows times
//       the F2 results, plus the chunk-end terms.
// Being independent per chunk, it runs at several workgroups per CU off the walk's critical path.
#include "mem_common.h"
#include "mem_params.h"
#include "seg_common.h"

namespace atlas {

constexpr int kScalarThreads = 256;
constexpr int kScalarWaves = kScalarThreads / kWave;

template <int CH>
struct BwdScalarSmem {
  static constexpr int SPM = CH + kHaloPad;
  static constexpr int LWR = ((CH + 2 + 15) / 16) * 16;   // rows of the F2 operand
  float Lm[CH][SPM + 1];
  float hS[SPM], hZ[SPM], fS[CH], fZ[CH];
  float gram[4];
  float Lw[LWR][CH + 1];      // window-weighted Lm rows (q < CH), hS (row CH), hZ (row CH + 1)
  float LWs[CH + 2][CH + 1];  // Lw C^T: rows q; row CH = from hS, row CH + 1 unused
  float LWz[CH + 2][CH + 1];  // Lw B^T: rows q; row CH = from hS, row CH + 1 = from hZ
  ChunkScalars<CH> sc;
  DecayTab<CH> tab;
  float B1[CH + 1];           // b_{t-1}, t = 0..CH
};

template <typename T, int CH>
__global__ __launch_bounds__(kScalarThreads) void k_bwd_scalar(const Geom g, const BwdPtrs<T> a,
                                                                 const BwdSegPtrs p) {
  typedef BwdScalarSmem<CH> Sm;
  typedef ScalarBlock<CH> SB;
  constexpr int SPM = Sm::SPM;
  __shared__ Sm sm;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int c = blockIdx.x, bh = blockIdx.y;
  const int H = g.H, e = g.e;
  const int t0 = c * g.Lc, L = min(g.T, t0 + g.Lc) - t0;
  const size_t tb = (size_t)bh * g.T, r0 = tb + t0;

  // ---- loads: the walk's inner products, the chunk's scalars and gates, a_{t-1} / kappa_{t-1}
  {
    const float* blk = p.scal + ((size_t)bh * g.nc + c) * SB::SIZE;
    for (int idx = tid; idx < CH * SPM; idx += kScalarThreads) sm.Lm[idx / SPM][idx % SPM] = blk[SB::LM + idx];
    for (int idx = tid; idx < SPM; idx += kScalarThreads) { sm.hS[idx] = blk[SB::HS + idx]; sm.hZ[idx] = blk[SB::HZ + idx]; }
    if (tid < CH) { sm.fS[tid] = blk[SB::FS + tid]; sm.fZ[tid] = blk[SB::FZ + tid]; }
    if (tid < 4) sm.gram[tid] = blk[SB::GRAM + tid];
    const float* rec = p.coef + ((size_t)bh * g.nc + c) * CoefRec<CH>::SIZE;
    for (int idx = tid; idx < 2 * CH + 4; idx += kScalarThreads) (&sm.sc.acoef[0])[idx] = rec[idx];
    if (tid < CH) {   // padded targets: alpha = beta = 1, eta = 0
      const bool ok = tid < L;
      const size_t rt = ok ? r0 + tid : r0;
      const T x_al = a.decay[rt], x_et = a.lr[rt], x_be = ((g.momentum && a.beta) ? a.beta : a.decay)[rt];
      sm.sc.alpha[tid] = ok ? to_f32(x_al) : 1.f;
      sm.sc.eta[tid] = ok ? to_f32(x_et) : 0.f;
      sm.sc.beta[tid] = ok ? (g.momentum ? to_f32(x_be) : 0.f) : 1.f;
    }
    const T* gp = a.gate ? a.gate : a.decay;
    if (g.gate_mode == GATE_TOKEN) {
      // the gate of each source; sources before the sequence (buffer products) count as gated
      for (int s = tid; s < SPM; s += kScalarThreads) {
        const int pg = t0 - H + s;
        const bool in = s < H + L;
        const T x = gp[(in && pg >= 0) ? tb + pg : r0];
        sm.sc.ug[s] = in ? (pg >= 0 ? to_f32(x) : 1.f) : 0.f;
      }
    } else if (g.gate_mode == GATE_LAG) {
      for (int idx = tid; idx < CH * e; idx += kScalarThreads) {
        const bool ok = idx / e < L;
        const T x = gp[ok ? r0 * e + idx : r0];
        sm.sc.wl[idx] = ok ? to_f32(x) : 0.f;
      }
    }
  }
  __syncthreads();

  // ---- decay tables (wave 0) | F1 (waves 1..)
  if (wave == 0) {
    decay_columns_wave<CH>(sm.tab, sm.sc, sm.B1);
  } else {
    for (int idx = tid - kWave; idx < (CH + 2) * CH; idx += kScalarThreads - kWave) {
      const int q = idx / CH, tq = idx % CH;
      const float* X = q < CH ? &sm.Lm[q][0] : (q == CH ? sm.hS : sm.hZ);
      float acc = 0.f;
      if (tq < L) {
        for (int j = 0; j < e; ++j) {
          const int s = tq + H - j;
          acc += src_w(g.gate_mode, sm.sc.ug[s], sm.sc.wl, e, tq, j) * X[s];
        }
      }
      sm.Lw[q][tq] = acc;
    }
  }
  __syncthreads();

  // ---- F2: the window-weighted recurrences along the chunk as GEMMs with the decay tables:
  //   LWz[q][t] = sum_t' B[t'+1][t] Lw[q][t'],   LWs[q][t] = sum_t' C[t'+1][t] Lw[q][t']
  {
    typedef MM<float> MF;
    constexpr int NRT = Sm::LWR / 16, NCT = CH / 16;
    for (int job = wave; job < 2 * NRT * NCT; job += kScalarWaves) {
      const int mat = job / (NRT * NCT), tile = job % (NRT * NCT);
      const int m0 = (tile / NCT) * 16, n0 = (tile % NCT) * 16;
      const float* tabp = mat == 0 ? &sm.tab.B[1][0] : &sm.tab.C[1][0];
      f32x4 acc = zero4();
#pragma unroll
      for (int k0 = 0; k0 < CH; k0 += MF::KS)
        acc = MF::mma(frag_ld<float>(&sm.Lw[0][0], CH + 1, 1, m0, k0), frag_ld<float>(tabp, 1, CH + 1, n0, k0), acc);
      float* dst = mat == 0 ? &sm.LWz[0][0] : &sm.LWs[0][0];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int q = m0 + 4 * (lane >> 4) + r;
        if (q < CH + 2) dst[q * (CH + 1) + n0 + (lane & 15)] = acc[r];
      }
    }
  }
  __syncthreads();

  // ---- F3: one wave per term (0: dalpha, 1: deta, 2: dbeta, 3 + j: dw[t, j]); lane = (q part, target t).
  //   The running products of the step-by-step adjoint are table entries: prod alpha = A[t+1][q-1],
  //   prod beta = B[t+1][q-1], the eta-mixed term = C[t+1][q-1] (zero for q - 1 < t).
  {
    constexpr int NQ = kWave / CH;
    constexpr int QPP = CH / NQ;
    const int t = lane % CH, part = lane / CH;
    const int nterm = 3 + (g.gate_mode != GATE_NONE ? e : 0);
    const float gss = sm.gram[0], gsz = sm.gram[1], gzz = sm.gram[2];
    const float am1 = sm.sc.acoef[t], km1 = sm.sc.kcoef[t], bm1 = sm.B1[t], b0 = sm.B1[t + 1];
    const float Aend = sm.tab.A[t + 1][CH - 1], Bend = sm.tab.B[t + 1][CH - 1], Cend = sm.tab.C[t + 1][CH - 1];
    for (int term = wave; term < nterm; term += kScalarWaves) {
      const float* W = term < 2 ? &sm.tab.A[t + 1][0] : &sm.tab.C[t + 1][0];
      const int sj = term >= 3 ? t + H - (term - 3) : 0;
      float acc = 0.f;
#pragma unroll 4
      for (int qq = 0; qq < QPP; ++qq) {
        const int q = part * QPP + qq;
        if (q >= 1) {
          float v;
          if (term == 0) v = am1 * sm.fS[q] - km1 * sm.fZ[q] - (t > 0 ? sm.LWs[q][t - 1] : 0.f);
          else if (term == 1) v = b0 * sm.fZ[q] + sm.LWz[q][t];
          else if (term == 2) v = bm1 * sm.fZ[q] + (t > 0 ? sm.LWz[q][t - 1] : 0.f);
          else v = sm.Lm[q][sj];
          acc += W[q - 1] * v;
        }
      }
#pragma unroll
      for (int off = CH; off < kWave; off <<= 1) acc += __shfl_xor(acc, off);
      if (part == 0 && t < L) {
        const size_t tt = r0 + t;
        if (term == 0) {
          const float hss_m1 = t > 0 ? sm.LWs[CH][t - 1] : 0.f;
          a.ddecay[tt] = from_f32<T>(acc + Aend * (am1 * gss - km1 * gsz - hss_m1));
        } else if (term == 1) {
          a.dlr[tt] = from_f32<T>(-(acc + Aend * (b0 * gsz + sm.LWz[CH][t])));
        } else if (term == 2) {
          if (g.momentum && a.dbeta) {
            const float hzs_m1 = t > 0 ? sm.LWz[CH][t - 1] : 0.f;
            const float hzz_m1 = t > 0 ? sm.LWz[CH + 1][t - 1] : 0.f;
            a.dbeta[tt] = from_f32<T>(Bend * (bm1 * gzz + hzz_m1) - Cend * (bm1 * gsz + hzs_m1) - acc);
          }
        } else {
          const int j = term - 3;
          const float v = Bend * sm.hZ[sj] - Cend * sm.hS[sj] - acc;
          if (g.gate_mode == GATE_LAG) a.dgate[tt * e + j] = from_f32<T>(v);
          else p.dw[tt * e + j] = v;
        }
      }
    }
  }
}

template <typename T, int CH>
hipError_t launch_bwd_scalar(const Geom& g, const BwdPtrs<T>& a, const BwdSegPtrs& p, hipStream_t stream) {
  prof_begin(KID_BWD_SCALAR, stream);
  hipLaunchKernelGGL((k_bwd_scalar<T, CH>), dim3(g.nc, g.BH), dim3(kScalarThreads), 0, stream, g, a, p);
  prof_end(KID_BWD_SCALAR, stream);
  return hipGetLastError();
}

#define ATLAS_INST_BWD_SCALAR(T, CH) \
  template hipError_t launch_bwd_scalar<T, CH>(const Geom&, const BwdPtrs<T>&, const BwdSegPtrs&, hipStream_t);

ATLAS_INST_BWD_SCALAR(bf16, 32)
ATLAS_INST_BWD_SCALAR(float, 16)

}  // namespace atlas
