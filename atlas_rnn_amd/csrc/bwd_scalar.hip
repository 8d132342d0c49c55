// bwd_scalar.hip - gradients of the per-token scalars (decay alpha, lr eta, momentum beta, window
// gates) of the chunked backward, one workgroup per backward chunk.
//
// Every scalar gradient is a sum over the chunk of decay-weighted inner products between the
// adjoint and the state. The reverse walk (k_bwd_seg) leaves those inner products per chunk in
// a ScalarBlock (Lm, hS, hZ, fS, fZ and the three Grams of the chunk-end adjoint with the
// chunk-start state); this kernel forms the chunk's decay tables and contracts them:
//   Lw  = X Wb    (X rows: Lm[q] for q < CH, hS, hZ; Wb: the band of window weights)
//   LWz = Lw Bsh, LWs = Lw Csh     (all three on the fp32 matrix cores)
//   then one wave per term (dalpha, deta, dbeta, dw[., j]): sums over q of table rows times
//   the products above, plus the chunk-end terms.
// Being independent per chunk, it runs at several workgroups per CU off the walk's critical path.
#include "mem_common.h"
#include "mem_params.h"
#include "seg_common.h"

namespace atlas {

constexpr int kScalarThreads = 512;
constexpr int kScalarWaves = kScalarThreads / kWave;

// Decay tables in shifted form (row t stands for the adjoint step after target t):
//   Ash[t][q] = prod_{r=t+1..q} alpha_r,  Bsh[t][q] = prod_{r=t+1..q} beta_r   (1 at q = t, 0 for q < t)
//   Csh[t][q] = sum_r Bsh[t][r] eta_r Ash[r][q]   (the eta-mixed momentum/decay term)
template <int CH>
struct BwdScalarSmem {
  static constexpr int SPM = CH + kHaloPad;
  static constexpr int LWR = ((CH + 2 + 15) / 16) * 16;   // rows of the window-weighted operand
  float X[LWR][SPM + 1];      // rows q < CH: Lm[q]; row CH: hS; row CH + 1: hZ; zero below
  float Ash[CH][CH + 1], Bsh[CH][CH + 1], Csh[CH][CH + 1];
  float Lw[LWR][CH + 1];      // X Wb: window-weighted rows
  union {
    float Wb[SPM][CH + 1];    // band of window weights: Wb[s][t] = w(t, t + H - s) (0 outside the window)
    struct {
      float LWs[CH + 2][CH + 1];   // Lw Csh (rows q <= CH + 1)
      float LWz[CH + 2][CH + 1];   // Lw Bsh
    } f;
  } u;
  float fS[CH], fZ[CH];
  float alpha[CH], eta[CH], beta[CH];
  float acoef[CH], kcoef[CH];
  float B1[CH + 1];           // b_{t-1} = prod_{r<t} beta_r
  float gram[4];
};

// C = A B over the 16 x 16 output tiles `job` of an M x N result (NT convention of MM<float>),
// A[m][k] at a[m * lda + k] (optionally scaled by s[k]), B[k][n] at b[k * ldb + n].
template <int K, bool SCALE>
__device__ __forceinline__ f32x4 tile_gemm_f32(const float* a, int lda, const float* b, int ldb, int m0, int n0,
                                               const float* s) {
  typedef MM<float> MF;
  f32x4 acc = zero4();
#pragma unroll
  for (int k0 = 0; k0 < K; k0 += MF::KS) {
    const float fa = SCALE ? frag_ld_kscaled<float>(a, lda, 1, m0, k0, s) : frag_ld<float>(a, lda, 1, m0, k0);
    acc = MF::mma(fa, frag_ld<float>(b, 1, ldb, n0, k0), acc);
  }
  return acc;
}

template <typename T, int CH>
__global__ __launch_bounds__(kScalarThreads) void k_bwd_scalar(const Geom g, const BwdPtrs<T> a,
                                                                 const BwdSegPtrs p) {
  if (geom_skip(g)) return;
  typedef BwdScalarSmem<CH> Sm;
  typedef ScalarBlock<CH> SB;
  constexpr int SPM = Sm::SPM, LWR = Sm::LWR;
  static_assert(SB::HS == CH * SPM && SB::HZ == SB::HS + SPM, "X rows are contiguous in the block");
  __shared__ Sm sm;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int c = blockIdx.x, bh = blockIdx.y;
  const int H = g.H, e = g.e;
  const int t0 = c * g.Lc, L = min(g.T, t0 + g.Lc) - t0;
  const size_t tb = (size_t)bh * g.T, r0 = tb + t0;

  // ---- loads: the walk's inner products, the scalars, the window band, a_{t-1} / kappa_{t-1}.
  // Every global load is issued (unrolled, from in-bounds addresses) before any LDS store.
  {
    const float* blk = p.scal + ((size_t)bh * g.nc + c) * SB::SIZE;
    constexpr int NX4 = (CH + 2) * SPM / 4;
    constexpr int NXI = (NX4 + kScalarThreads - 1) / kScalarThreads;
    constexpr int NWI = (SPM * CH + kScalarThreads - 1) / kScalarThreads;
    static_assert(((CH + 2) * SPM) % 4 == 0 && SPM % 4 == 0, "float4 rows");
    const float* rec = p.coef + ((size_t)bh * g.nc + c) * CoefRec<CH>::SIZE;
    const T* gp = a.gate ? a.gate : a.decay;
    float4 xv[NXI];
#pragma unroll
    for (int u = 0; u < NXI; ++u) {
      const int v = tid + u * kScalarThreads;
      xv[u] = reinterpret_cast<const float4*>(blk)[v < NX4 ? v : 0];
    }
    const int ts = tid < CH ? tid : 0;
    const bool ok_t = tid < L;
    const size_t rt = ok_t ? r0 + ts : r0;
    const float x_fs = blk[SB::FS + ts], x_fz = blk[SB::FZ + ts], x_gr = blk[SB::GRAM + (tid & 3)];
    const float x_ac = rec[ts], x_kc = rec[CH + ts];
    const T x_al = a.decay[rt], x_et = a.lr[rt], x_be = ((g.momentum && a.beta) ? a.beta : a.decay)[rt];
    // Wb[s][t]: weight of source s in the window sum of target t (j = t + H - s). Token gates weight
    // the source (sources before the sequence are buffer products, already gated: weight 1).
    T xw[NWI];
    bool in_w[NWI], buf_w[NWI];
#pragma unroll
    for (int u = 0; u < NWI; ++u) {
      const int idx = tid + u * kScalarThreads;
      const int s = idx / CH, t = idx % CH, j = t + H - s;
      in_w[u] = idx < SPM * CH && t < L && j >= 0 && j < e;
      const int ps = t0 - H + s;
      buf_w[u] = ps < 0;
      size_t off = r0;
      if (g.gate_mode == GATE_TOKEN && in_w[u] && ps >= 0) off = tb + ps;
      if (g.gate_mode == GATE_LAG && in_w[u]) off = (r0 + t) * e + j;
      xw[u] = gp[off];
    }
#pragma unroll
    for (int u = 0; u < NXI; ++u) {
      const int v = tid + u * kScalarThreads;
      if (v < NX4) {
        const int q = (4 * v) / SPM, s = (4 * v) % SPM;
        sm.X[q][s] = xv[u].x; sm.X[q][s + 1] = xv[u].y; sm.X[q][s + 2] = xv[u].z; sm.X[q][s + 3] = xv[u].w;
      }
    }
    for (int idx = tid; idx < (LWR - CH - 2) * SPM; idx += kScalarThreads) sm.X[CH + 2 + idx / SPM][idx % SPM] = 0.f;
    if (tid < CH) {   // padded targets: alpha = beta = 1, eta = 0
      sm.fS[tid] = x_fs; sm.fZ[tid] = x_fz;
      sm.acoef[tid] = x_ac; sm.kcoef[tid] = x_kc;
      sm.alpha[tid] = ok_t ? to_f32(x_al) : 1.f;
      sm.eta[tid] = ok_t ? to_f32(x_et) : 0.f;
      sm.beta[tid] = ok_t ? (g.momentum ? to_f32(x_be) : 0.f) : 1.f;
    }
    if (tid < 4) sm.gram[tid] = x_gr;
#pragma unroll
    for (int u = 0; u < NWI; ++u) {
      const int idx = tid + u * kScalarThreads;
      if (idx < SPM * CH) {
        float w = in_w[u] ? 1.f : 0.f;
        if (g.gate_mode == GATE_TOKEN) w = in_w[u] ? (buf_w[u] ? 1.f : to_f32(xw[u])) : 0.f;
        else if (g.gate_mode == GATE_LAG) w = in_w[u] ? to_f32(xw[u]) : 0.f;
        sm.u.Wb[idx / CH][idx % CH] = w;
      }
    }
  }
  __syncthreads();

  // ---- decay tables: one row per lane, serial along q (wave 0: alpha, wave 1: beta and b_{t-1})
  //      | window sums Lw = X Wb on the matrix cores (the other waves)
  if (wave < 2) {
    const int t = lane;
    const float* f = wave == 0 ? sm.alpha : sm.beta;
    const float fv = f[lane < CH ? lane : 0];
    float* row = wave == 0 ? &sm.Ash[0][0] : &sm.Bsh[0][0];
    float x = 1.f;
#pragma unroll
    for (int q = 0; q < CH; ++q) {
      const float fq = lane_bcast(fv, q);
      if (q > t) x *= fq;
      if (t < CH) row[t * (CH + 1) + q] = q >= t ? x : 0.f;
    }
    if (wave == 1 && lane == CH) {   // b_{t-1}: the product from the chunk start
      float b = 1.f;
      sm.B1[0] = 1.f;
#pragma unroll
      for (int q = 0; q < CH; ++q) {
        b *= lane_bcast(fv, q);
        sm.B1[q + 1] = b;
      }
    }
  } else {
    constexpr int NRT = LWR / 16, NCT = CH / 16;
    for (int job = wave - 2; job < NRT * NCT; job += kScalarWaves - 2) {
      const int m0 = (job / NCT) * 16, n0 = (job % NCT) * 16;
      const f32x4 acc = tile_gemm_f32<SPM, false>(&sm.X[0][0], SPM + 1, &sm.u.Wb[0][0], CH + 1, m0, n0, nullptr);
#pragma unroll
      for (int r = 0; r < 4; ++r) sm.Lw[m0 + 4 * (lane >> 4) + r][n0 + (lane & 15)] = acc[r];
    }
  }
  __syncthreads();

  // ---- Csh = Bsh diag(eta) Ash | LWz = Lw Bsh
  {
    constexpr int NCT = CH / 16, NRT = LWR / 16;
    constexpr int NJ_C = NCT * NCT, NJ = NJ_C + NRT * NCT;
    for (int job = wave; job < NJ; job += kScalarWaves) {
      if (job < NJ_C) {
        const int m0 = (job / NCT) * 16, n0 = (job % NCT) * 16;
        const f32x4 acc = tile_gemm_f32<CH, true>(&sm.Bsh[0][0], CH + 1, &sm.Ash[0][0], CH + 1, m0, n0, sm.eta);
#pragma unroll
        for (int r = 0; r < 4; ++r) sm.Csh[m0 + 4 * (lane >> 4) + r][n0 + (lane & 15)] = acc[r];
      } else {
        const int jb = job - NJ_C;
        const int m0 = (jb / NCT) * 16, n0 = (jb % NCT) * 16;
        const f32x4 acc = tile_gemm_f32<CH, false>(&sm.Lw[0][0], CH + 1, &sm.Bsh[0][0], CH + 1, m0, n0, nullptr);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int q = m0 + 4 * (lane >> 4) + r;
          if (q < CH + 2) sm.u.f.LWz[q][n0 + (lane & 15)] = acc[r];
        }
      }
    }
  }
  __syncthreads();
  // ---- LWs = Lw Csh
  {
    constexpr int NCT = CH / 16, NRT = LWR / 16;
    for (int job = wave; job < NRT * NCT; job += kScalarWaves) {
      const int m0 = (job / NCT) * 16, n0 = (job % NCT) * 16;
      const f32x4 acc = tile_gemm_f32<CH, false>(&sm.Lw[0][0], CH + 1, &sm.Csh[0][0], CH + 1, m0, n0, nullptr);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int q = m0 + 4 * (lane >> 4) + r;
        if (q < CH + 2) sm.u.f.LWs[q][n0 + (lane & 15)] = acc[r];
      }
    }
  }
  __syncthreads();

  // ---- one wave per term (0: dalpha, 1: deta, 2: dbeta, 3 + j: dw[t, j]); lane = (q part, target t).
  //   The running products of the step-by-step adjoint are table entries: prod alpha = Ash[t][q-1],
  //   prod beta = Bsh[t][q-1], the eta-mixed term = Csh[t][q-1] (zero for q - 1 < t).
  {
    constexpr int NQ = kWave / CH;
    constexpr int QPP = CH / NQ;
    const int t = lane % CH, part = lane / CH;
    const int nterm = 3 + (g.gate_mode != GATE_NONE ? e : 0);
    const float gss = sm.gram[0], gsz = sm.gram[1], gzz = sm.gram[2];
    const float am1 = sm.acoef[t], km1 = sm.kcoef[t], bm1 = sm.B1[t], b0 = sm.B1[t + 1];
    const float Aend = sm.Ash[t][CH - 1], Bend = sm.Bsh[t][CH - 1], Cend = sm.Csh[t][CH - 1];
    for (int term = wave; term < nterm; term += kScalarWaves) {
      const float* W = term < 2 ? &sm.Ash[t][0] : &sm.Csh[t][0];
      const int sj = term >= 3 ? t + H - (term - 3) : 0;
      float acc = 0.f;
#pragma unroll 4
      for (int qq = 0; qq < QPP; ++qq) {
        const int q = part * QPP + qq;
        if (q >= 1) {
          float v;
          if (term == 0) v = am1 * sm.fS[q] - km1 * sm.fZ[q] - (t > 0 ? sm.u.f.LWs[q][t - 1] : 0.f);
          else if (term == 1) v = b0 * sm.fZ[q] + sm.u.f.LWz[q][t];
          else if (term == 2) v = bm1 * sm.fZ[q] + (t > 0 ? sm.u.f.LWz[q][t - 1] : 0.f);
          else v = sm.X[q][sj];
          acc += W[q - 1] * v;
        }
      }
#pragma unroll
      for (int off = CH; off < kWave; off <<= 1) acc += __shfl_xor(acc, off);
      if (part == 0 && t < L) {
        const size_t tt = r0 + t;
        if (term == 0) {
          const float hss_m1 = t > 0 ? sm.u.f.LWs[CH][t - 1] : 0.f;
          a.ddecay[tt] = from_f32<T>(acc + Aend * (am1 * gss - km1 * gsz - hss_m1));
        } else if (term == 1) {
          a.dlr[tt] = from_f32<T>(-(acc + Aend * (b0 * gsz + sm.u.f.LWz[CH][t])));
        } else if (term == 2) {
          if (g.momentum && a.dbeta) {
            const float hzs_m1 = t > 0 ? sm.u.f.LWz[CH][t - 1] : 0.f;
            const float hzz_m1 = t > 0 ? sm.u.f.LWz[CH + 1][t - 1] : 0.f;
            a.dbeta[tt] = from_f32<T>(Bend * (bm1 * gzz + hzz_m1) - Cend * (bm1 * gsz + hzs_m1) - acc);
          }
        } else {
          const int j = term - 3;
          const float v = Bend * sm.X[CH + 1][sj] - Cend * sm.X[CH][sj] - acc;
          if (g.gate_mode == GATE_LAG) a.dgate[tt * e + j] = from_f32<T>(v);
          else p.dw[tt * e + j] = v;
        }
      }
    }
  }
}

template <typename T, int CH>
hipError_t launch_bwd_scalar(const Geom& g, const BwdPtrs<T>& a, const BwdSegPtrs& p, hipStream_t stream) {
  prof_name(KID_BWD_SCALAR, "k_bwd_scalar");
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
