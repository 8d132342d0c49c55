// seg_bwd.hip - segment-parallel backward pass of the chunked memory recurrence (gfx950).
//
// Same segments as the forward pass (one workgroup per (segment, bh), 8 waves), chunks of Lb tokens
// (Lb <= 32 for bf16, <= 16 for fp32 so that every operand of a chunk fits in LDS):
//   k_bwd_seg_agg : reverse walk of the segment's chunks from a zero adjoint -> adjoint aggregate
//                   (the transposed 2x2 transition and the local chunk-start adjoint L, K):
//                     dS_in = a dS_end + sum_t a_{t-1} dy_t psi_t^T
//                     dZ_in = b dZ_end - kappa dS_end - sum_t kappa_{t-1} dy_t psi_t^T
//   k_bwd_seg_scan: one thread per state element folds the aggregates from the last segment back,
//                   writing the adjoint (dS, dZ) at every segment end.
//   k_bwd_seg     : starts from the adjoint at its segment end and walks the segment's chunks in
//                   reverse forming every gradient of each chunk in closed form (see k_bwd_seg's
//                   phase comments) while carrying (dS, dZ) and the halo gradients of the previous
//                   chunk's last e-1 tokens.
//   k_bwd_seg_fixup : merges the partial (dv, dphi) of tokens whose window crosses a segment boundary,
//                   adds the d buffer_out terms, reduces token-gate gradients and (without d buffer_out)
//                   the dS_ref partials; with d buffer_out k_seg_reduce_dsref reduces them afterwards.
#include <type_traits>

#include "mem_common.h"
#include "mem_params.h"
#include "seg_common.h"
#include "seg_fixup.h"

namespace atlas {

template <typename T, int CH>
hipError_t launch_bwd_scalar(const Geom& g, const BwdPtrs<T>& a, const BwdSegPtrs& p, hipStream_t stream);

// ---------------------------------------------------------------------------------------------
// adjoint aggregates
// ---------------------------------------------------------------------------------------------
template <typename T, int CH, int D>
struct BwdAggSmem {
  // The aggregates over the forward's 64-token chunks (the specialised path) stage dy pre-scaled
  // by both coefficients, once per chunk, instead of scaling every fragment as it is used (four
  // waves share each dy fragment); the general path's chunk lengths keep the per-fragment scaling.
  static constexpr bool kPre = CH == 64;
  struct PreDy {
    alignas(16) T a[CH][D + 8];   // a_{t-1} dy_t, rounded to T
    alignas(16) T k[CH][D + 8];   // kappa_{t-1} dy_t, rounded to T
  };
  struct NoDy {};
  alignas(16) T psi[CH][D + 8];
  alignas(16) T dy[CH][D + 8];                 // unscaled (per-fragment scaling)
  alignas(16) float coef[2 * CH + 4];          // a_{t-1}, kappa_{t-1}, (a, kappa, b) of the chunk
  typename std::conditional<kPre, PreDy, NoDy>::type pre;
};

// Register prefetch of one chunk for the adjoint aggregates: psi (vectors 0 .. NV-1) or dy
// (vectors NV .. 2 NV-1) rows, 8 features per vector, NVT vectors per thread, the coefficients
// a_{t-1}, kappa_{t-1} of each dy vector's token, and the head of the coefficient record. The dy
// rows are stored scaled by both coefficients (once per chunk, instead of once per fragment use).
template <int N>
struct AggPreW {   // coefficients of the dy vectors (pre-scaled staging only)
  float a[N], k[N];
};
struct AggNoW {};

template <typename T, int CH, int D>
struct BwdAggPrefetch
    : std::conditional<BwdAggSmem<T, CH, D>::kPre, AggPreW<(2 * (CH * D / 8) + kSegThreads - 1) / kSegThreads>,
                       AggNoW>::type {
  static constexpr int NV = CH * D / 8;
  static constexpr int NVT = (2 * NV + kSegThreads - 1) / kSegThreads;
  static constexpr int NC4 = (2 * CH + 4) / 4;
  static_assert((2 * CH + 4) % 4 == 0 && NC4 <= kSegThreads, "record head");
  Vec8<T> x[NVT];
  float4 rc;
  bool ok[NVT];
  __device__ __forceinline__ void load(const Geom& g, const BwdPtrs<T>& a, const float* rec, size_t tb, int c,
                                       int tid) {
    const int t0 = c * g.Lc, L = min(g.T, t0 + g.Lc) - t0;
#pragma unroll
    for (int u = 0; u < NVT; ++u) {
      const int vi = tid + u * kSegThreads;
      const int v = vi < NV ? vi : vi - NV;
      const int t = v / (D / 8), c8 = v % (D / 8);
      const T* src = (vi < NV || !a.dy) ? a.q : a.dy;
      ok[u] = vi < 2 * NV && t < L && (vi < NV || a.dy);
      x[u] = vec8_load(src + (tb + t0 + (ok[u] ? t : 0)) * D + c8 * 8);
      if constexpr (BwdAggSmem<T, CH, D>::kPre) {
        const int tc = t < CH ? t : 0;
        this->a[u] = rec[tc];
        this->k[u] = rec[CH + tc];
      }
    }
    rc = reinterpret_cast<const float4*>(rec)[tid < NC4 ? tid : 0];
  }
  template <typename Sm>
  __device__ __forceinline__ void store(const Geom& g, Sm& sm, int tid) const {
#pragma unroll
    for (int u = 0; u < NVT; ++u) {
      const int vi = tid + u * kSegThreads;
      if (vi < 2 * NV) {
        const int v = vi < NV ? vi : vi - NV;
        const int t = v / (D / 8), c8 = v % (D / 8);
        Vec8<T> y = x[u].masked(ok[u]);
        if (vi < NV) {
          if (g.map_mode == MAP_ELEMENTWISE) y = y.mapped(g.map_deg);
          y.store(&sm.psi[t][c8 * 8]);
        } else {
          if constexpr (Sm::kPre) {
            y.store_scaled(&sm.pre.a[t][c8 * 8], this->a[u]);
            y.store_scaled(&sm.pre.k[t][c8 * 8], this->k[u]);
          } else {
            y.store(&sm.dy[t][c8 * 8]);
          }
        }
      }
    }
    if (tid < NC4) reinterpret_cast<float4*>(sm.coef)[tid] = rc;
  }
};

// The same staging for the forward's 64-token chunks at d = 64 (pre-scaled dy, one psi and one dy
// vector per thread: psi row tid >> 3, dy row tid >> 3, 8 features at 8 (tid & 7)), with the
// per-thread row pointers and offsets formed once per launch instead of once per chunk.
template <typename T, int CH, int D>
struct BwdAggFastPf {
  static constexpr int NC4 = (2 * CH + 4) / 4;
  Vec8<T> xq, xd;
  float wa, wk;
  float4 rc;
  bool okq, okd;
  const T* pq;   // psi row t of chunk 0 (rows past T read the sequence's first row, masked)
  const T* pd;
  const T* pq0;
  const T* pd0;
  int t;
  __device__ __forceinline__ void init(const BwdPtrs<T>& a, size_t tb, int tid) {
    t = tid >> 3;
    const int c8 = tid & 7;
    pq0 = a.q + tb * D + c8 * 8;
    pd0 = (a.dy ? a.dy : a.q) + tb * D + c8 * 8;
    pq = pq0 + (size_t)t * D;
    pd = pd0 + (size_t)t * D;
  }
  __device__ __forceinline__ void load(const Geom& g, const BwdPtrs<T>& a, const float* rec, size_t, int c, int tid) {
    const int t0 = c * CH, L = min(g.T, t0 + CH) - t0;
    okq = t < L;
    okd = okq && a.dy != nullptr;
    xq = vec8_load(okq ? pq + (size_t)t0 * D : pq0);
    xd = vec8_load(okd ? pd + (size_t)t0 * D : pd0);
    wa = rec[t];
    wk = rec[CH + t];
    rc = reinterpret_cast<const float4*>(rec)[tid < NC4 ? tid : 0];
  }
  template <typename Sm>
  __device__ __forceinline__ void store(const Geom& g, Sm& sm, int tid) const {
    const int c8 = tid & 7;
    Vec8<T> y = xq.masked(okq);
    if (g.map_mode == MAP_ELEMENTWISE) y = y.mapped(g.map_deg);
    y.store(&sm.psi[t][c8 * 8]);
    const Vec8<T> z = xd.masked(okd);
    z.store_scaled(&sm.pre.a[t][c8 * 8], wa);
    z.store_scaled(&sm.pre.k[t][c8 * 8], wk);
    if (tid < NC4) reinterpret_cast<float4*>(sm.coef)[tid] = rc;
  }
};

// Adjoint aggregate of one segment: walks its chunks in reverse from a zero adjoint,
//   lam <- a_end lam + sum_t a_{t-1} dy_t psi_t^T,   mu <- b_end mu - kappa_end lam - sum_t kappa_{t-1} dy_t psi_t^T,
// with the next chunk's inputs prefetched into registers while the current one computes.
template <typename T, int CH, int D>
__global__ __launch_bounds__(kSegThreads) void k_bwd_seg_agg(const Geom g, const BwdPtrs<T> a, const SegGeom sg,
                                                               const BwdSegPtrs p) {
  if (geom_skip(g)) return;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  typedef BwdAggSmem<T, CH, D> Sm;
  Sm& sm = *reinterpret_cast<Sm*>(smem_raw);
  constexpr int NTD = D / 16;
  constexpr int NT2 = (NTD * NTD + kSegWaves - 1) / kSegWaves;   // state tiles per wave
  // pre-scaled dy with two tiles per wave: wave w owns row tile w >> 1, column tiles 2 (w & 1) + j
  constexpr bool kPair = Sm::kPre && NTD * NTD == 2 * kSegWaves;
  typedef MM<T> M;
  const int seg = blockIdx.x, bh = blockIdx.y;
  const size_t tb = (size_t)bh * g.T;
  const int c_begin = seg * sg.G, c_end = min(g.nc, c_begin + sg.G);
  const float* rec_row = p.coef + (size_t)bh * g.nc * CoefRec<CH>::SIZE;
  float lam[NT2][4], mu[NT2][4];
#pragma unroll
  for (int j = 0; j < NT2; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) { lam[j][r] = 0.f; mu[j][r] = 0.f; }
  float pa = 1.f, pk = 0.f, pb = 1.f;
  constexpr bool kFast = Sm::kPre && D == 64 && CH * D / 8 == kSegThreads;
  typename std::conditional<kFast, BwdAggFastPf<T, CH, D>, BwdAggPrefetch<T, CH, D>>::type pf;
  if constexpr (kFast) pf.init(a, tb, threadIdx.x);
  if (c_begin < c_end) pf.load(g, a, rec_row + (size_t)(c_end - 1) * CoefRec<CH>::SIZE, tb, c_end - 1, threadIdx.x);
  for (int c = c_end - 1; c >= c_begin; --c) {
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & (kWave - 1), wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    __syncthreads();
    pf.store(g, sm, tid);
    __syncthreads();
    if (c - 1 >= c_begin) pf.load(g, a, rec_row + (size_t)(c - 1) * CoefRec<CH>::SIZE, tb, c - 1, tid);
    const float ae = sm.coef[2 * CH], ke = sm.coef[2 * CH + 1], be = sm.coef[2 * CH + 2];
    if constexpr (kPair) {
      // the wave's two tiles share their rows: the scaled dy fragments are read once per k-step
      const int m0 = (wave >> 1) * 16;
      f32x4 aa[2], ak[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) { aa[j] = zero4(); ak[j] = zero4(); }
#pragma unroll
      for (int k0 = 0; k0 < CH; k0 += M::KS) {
        const typename M::frag fa = frag_ld_tr<T>(&sm.pre.a[0][0], D + 8, m0, k0);
        const typename M::frag fk = frag_ld_tr<T>(&sm.pre.k[0][0], D + 8, m0, k0);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const typename M::frag fb = frag_ld_tr<T>(&sm.psi[0][0], D + 8, 16 * (2 * (wave & 1) + j), k0);
          aa[j] = M::mma(fa, fb, aa[j]);
          ak[j] = M::mma(fk, fb, ak[j]);
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float l_out = lam[j][r];
          lam[j][r] = ae * l_out + aa[j][r];
          mu[j][r] = g.momentum ? (be * mu[j][r] - ke * l_out - ak[j][r]) : 0.f;
        }
    }
#pragma unroll
    for (int j = 0; j < (kPair ? 0 : NT2); ++j) {
      const int tile = min(wave + kSegWaves * j, NTD * NTD - 1);
      const bool valid = (NTD * NTD) % kSegWaves == 0 || wave + kSegWaves * j < NTD * NTD;
      const int m0 = (tile / NTD) * 16, n0 = (tile % NTD) * 16;
      f32x4 aa = zero4(), ak = zero4();
#pragma unroll
      for (int k0 = 0; k0 < CH; k0 += M::KS) {
        const typename M::frag fb = frag_ld_tr<T>(&sm.psi[0][0], D + 8, n0, k0);
        if constexpr (Sm::kPre) {
          aa = M::mma(frag_ld_tr<T>(&sm.pre.a[0][0], D + 8, m0, k0), fb, aa);
          ak = M::mma(frag_ld_tr<T>(&sm.pre.k[0][0], D + 8, m0, k0), fb, ak);
        } else {
          const typename M::frag fd = frag_ld_tr<T>(&sm.dy[0][0], D + 8, m0, k0);
          const int kb = k0 + (lane >> 4) * M::KL;
          aa = M::mma(frag_scale<T>(fd, &sm.coef[kb]), fb, aa);
          ak = M::mma(frag_scale<T>(fd, &sm.coef[CH + kb]), fb, ak);
        }
      }
      if (valid) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float l_out = lam[j][r];
          lam[j][r] = ae * l_out + aa[r];
          mu[j][r] = g.momentum ? (be * mu[j][r] - ke * l_out - ak[r]) : 0.f;
        }
      }
    }
    const float na = pa * ae, nk = pa * ke + pk * be;
    pb = pb * be; pa = na; pk = nk;
  }
  const int lane = lane_id(), wave = wave_id();
  float* ag = p.adj_agg + ((size_t)bh * sg.nseg + seg) * sg.agg_stride;
#pragma unroll
  for (int j = 0; j < NT2; ++j) {
    const int tile = kPair ? (wave >> 1) * NTD + 2 * (wave & 1) + j : wave + kSegWaves * j;
    if (tile >= NTD * NTD) continue;
    const int m0 = (tile / NTD) * 16, n0 = (tile % NTD) * 16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = m0 + 4 * (lane >> 4) + r, k = n0 + (lane & 15);
      ag[(size_t)i * D + k] = lam[j][r];
      ag[(size_t)D * D + (size_t)i * D + k] = mu[j][r];
    }
  }
  if (threadIdx.x == 0) { ag[2 * D * D] = pa; ag[2 * D * D + 1] = pk; ag[2 * D * D + 2] = pb; }
}

// ---------------------------------------------------------------------------------------------
// main reverse walk
// ---------------------------------------------------------------------------------------------
template <typename T, int CH, int D>
struct BwdSegSmem {
  static constexpr int SPM = CH + kHaloPad;
  static constexpr bool kStatesInLds = sizeof(T) == 2;   // fp32 reads S_in / Z_in from the saved chunk states
  // adjoint at the chunk end and the chunk-start state, transposed: X^T[k][i] = X[i][k]
  alignas(16) T sref[D][D + 8];
  alignas(16) T dSeT[D][D + 8];
  alignas(16) T dZeT[D][D + 8];
  alignas(16) T SinT[kStatesInLds ? D : 1][D + 8];
  alignas(16) T ZinT[kStatesInLds ? D : 1][D + 8];
  T phi[SPM][D + 8];
  T psi[CH][D + 8];
  T dy[CH][D + 8];
  T deltaT[SPM][D + 8];    // v_s staged by the loads, then delta^T[s][i]
  struct {
    T QT[SPM][CH + 8];   // Q^T[s][q],  Q[q][s] = Ws[s, q-1] (psi_q . phi_s)
    T Qp[CH][SPM + 8];   // Q'[q][s] = Ws[s, q-1] (dy_q . delta_s)
    T QpT[SPM][CH + 8];
    alignas(16) T dDT[SPM][D + 8];   // dDelta^T[s][i]
  } g;
  T wsh[CH][SPM + 8];      // Ws[s, tau-1]
  float Lm[CH][SPM + 1];   // (dy_q . delta_s)(psi_q . phi_s)
  ChunkScalars<CH> sc;
  float hS[SPM], hZ[SPM], fS[CH], fZ[CH];
  float gram[4];
  float red[kSegWaves][4][4];   // per wave and lane row: partial Grams
  // followed by the halo carry: float carry[2][H][2 * D] (dynamic size)
};

// Register prefetch of one backward chunk's inputs (issued one chunk ahead of its use): k, v of
// the sources, q, dy of the targets, the scalars and gates, the coefficient record, the Ws[s, t-1]
// block and the saved chunk-start state tiles of this wave. Every load is unconditional from
// an in-bounds address; masks are applied in store().
template <typename T, int CH, int D>
struct BwdPrefetch {
  static constexpr int SPM = CH + kHaloPad;
  static constexpr int NTD = D / 16;
  static constexpr int NT2 = (NTD * NTD + kSegWaves - 1) / kSegWaves;
  static constexpr int NVS = (SPM * (D / 8) + kSegThreads - 1) / kSegThreads;
  static constexpr int NVT = (CH * (D / 8) + kSegThreads - 1) / kSegThreads;
  static constexpr int REC4 = CoefRec<CH>::SIZE / 4;
  static constexpr int NV_WSH = (CH * SPM / 8 + kSegThreads - 1) / kSegThreads;
  Vec8<T> rk[NVS], rv[NVS], rq[NVT], rd[NVT], wsv[NV_WSH];
  float rc0, rc1, rc2, rc3;
  unsigned okS, okT;
  float s_in[NT2][4], z_in[NT2][4];   // raw chunk-start state (saved by the forward), this wave's tiles

  __device__ __forceinline__ void load(const Geom& g, const BwdPtrs<T>& a, const BwdSegPtrs& p, int bh, int c,
                                       const float* Sin_g, int tid, int lane, int wave) {
    const int H = g.H;
    const size_t tb = (size_t)bh * g.T;
    const int t0 = c * g.Lc, L = min(g.T, t0 + g.Lc) - t0;
    const size_t r0 = tb + t0;
    okS = 0; okT = 0;
#pragma unroll
    for (int j = 0; j < NVS; ++j) {
      const int idx = tid + j * kSegThreads;
      const int s = idx / (D / 8), c8 = idx % (D / 8);
      const int pp = t0 - H + s;
      const bool ok = s < SPM && s < H + L && pp >= 0;
      const size_t row = ok ? tb + pp : r0;
      rk[j] = vec8_load(a.k + row * D + c8 * 8);
      rv[j] = vec8_load(a.v + row * D + c8 * 8);
      okS |= (ok ? 1u : 0u) << j;
    }
    const T* dyp = a.dy ? a.dy : a.q;
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
      const int idx = tid + j * kSegThreads;
      const int t = idx / (D / 8), c8 = idx % (D / 8);
      const bool ok = t < L;
      const size_t row = ok ? r0 + t : r0;
      rq[j] = vec8_load(a.q + row * D + c8 * 8);
      rd[j] = vec8_load(dyp + row * D + c8 * 8);
      okT |= (ok ? 1u : 0u) << j;
    }
    {
      const float4 r4 = reinterpret_cast<const float4*>(p.coef + ((size_t)bh * g.nc + c) * CoefRec<CH>::SIZE)[tid < REC4 ? tid : 0];
      rc0 = r4.x; rc1 = r4.y; rc2 = r4.z; rc3 = r4.w;
    }
    const T* wsh_c = reinterpret_cast<const T*>(p.wsh) + ((size_t)bh * g.nc + c) * CH * SPM;
#pragma unroll
    for (int j = 0; j < NV_WSH; ++j) {
      const int v = tid + j * kSegThreads;
      wsv[j] = vec8_load(wsh_c + (size_t)(v < CH * SPM / 8 ? v : 0) * 8);
    }
    const float* Zin_g = Sin_g + (size_t)D * D;
#pragma unroll
    for (int j = 0; j < NT2; ++j) {
      const int tile = min(wave + kSegWaves * j, NTD * NTD - 1);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = (tile / NTD) * 16 + 4 * (lane >> 4) + r, k = (tile % NTD) * 16 + (lane & 15);
        s_in[j][r] = Sin_g[(size_t)i * D + k];
        z_in[j][r] = Zin_g[(size_t)i * D + k];
      }
    }
  }

  // chunk inputs -> LDS (the states are consumed by the caller)
  template <typename Sm>
  __device__ __forceinline__ void store(const Geom& g, const BwdPtrs<T>& a, Sm& sm, int tid) {
#pragma unroll
    for (int j = 0; j < NVS; ++j) {
      const int idx = tid + j * kSegThreads;
      const int s = idx / (D / 8), c8 = idx % (D / 8);
      if (s < SPM) {
        const bool ok = (okS >> j) & 1u;
        Vec8<T> x = rk[j].masked(ok);
        if (g.map_mode == MAP_ELEMENTWISE) x = x.mapped(g.map_deg);
        x.store(&sm.phi[s][c8 * 8]);
        rv[j].masked(ok).store(&sm.deltaT[s][c8 * 8]);
      }
    }
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
      const int idx = tid + j * kSegThreads;
      const int t = idx / (D / 8), c8 = idx % (D / 8);
      if (t < CH) {
        const bool ok = (okT >> j) & 1u;
        Vec8<T> x = rq[j].masked(ok);
        if (g.map_mode == MAP_ELEMENTWISE) x = x.mapped(g.map_deg);
        x.store(&sm.psi[t][c8 * 8]);
        rd[j].masked(ok && a.dy).store(&sm.dy[t][c8 * 8]);
      }
    }
    if (tid < REC4) reinterpret_cast<float4*>(&sm.sc.acoef[0])[tid] = make_float4(rc0, rc1, rc2, rc3);
#pragma unroll
    for (int j = 0; j < NV_WSH; ++j) {
      const int v = tid + j * kSegThreads;
      if (v < CH * SPM / 8) wsv[j].store(&sm.wsh[(v * 8) / SPM][(v * 8) % SPM]);
    }
    if (tid < CH) { sm.fS[tid] = 0.f; sm.fZ[tid] = 0.f; }
    for (int s = tid; s < SPM; s += kSegThreads) { sm.hS[s] = 0.f; sm.hZ[s] = 0.f; }
  }
};

template <typename T, int CH, int D>
__global__ __launch_bounds__(kSegThreads) void k_bwd_seg(const Geom g, const BwdPtrs<T> a, const SegGeom sg,
                                                           const BwdSegPtrs p) {
  if (geom_skip(g)) return;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  typedef BwdSegSmem<T, CH, D> Sm;
  constexpr int SPM = Sm::SPM;
  constexpr bool SIL = Sm::kStatesInLds;
  constexpr int NTD = D / 16;
  constexpr int NT2 = (NTD * NTD + kSegWaves - 1) / kSegWaves;   // owned state tiles per wave
  typedef MM<T> M;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int seg = blockIdx.x, bh = blockIdx.y;
  const int H = g.H, e = g.e;
  constexpr int NTS = SPM / 16, NTC = CH / 16;
  static_assert(SPM <= 64, "backward source tile: coefficient lanes 0..63, decay columns 64..64+CH");
  const size_t tb = (size_t)bh * g.T;
  const size_t sb = (size_t)bh * D * D;
  const int c_begin = seg * sg.G, c_end = min(g.nc, c_begin + sg.G);
  // the segment's last H tokens: their partial (dv, dphi) goes to tail_part (merged by the fixup with the
  // next segment's halo and the d buffer_out terms)
  const int seg_tail0 = min(g.T, c_end * g.Lc) - H;
  const float* rw = p.rw + (size_t)bh * g.nc * 2 * D * D;   // raw chunk-start states of this row

  // ---- 1. adjoint at the segment end (owned tiles: wave + 8 j)
  float dS[NT2][4], dZ[NT2][4], dsr[NT2][4];
  {
    const float* sa = p.seg_adj + ((size_t)bh * sg.nseg + seg) * 2 * D * D;
#pragma unroll
    for (int j = 0; j < NT2; ++j) {
      const int tile = wave + kSegWaves * j;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        dS[j][r] = 0.f; dZ[j][r] = 0.f; dsr[j][r] = 0.f;
        if (tile < NTD * NTD) {
          const int i = (tile / NTD) * 16 + 4 * (lane >> 4) + r, k = (tile % NTD) * 16 + (lane & 15);
          dS[j][r] = sa[(size_t)i * D + k];
          dZ[j][r] = sa[(size_t)D * D + (size_t)i * D + k];
        }
      }
    }
  }

  Sm& sm = *reinterpret_cast<Sm*>(smem_raw);
  float* carry = reinterpret_cast<float*>(smem_raw + carry_offset<Sm>());   // [2][H][2D], 16-byte aligned
  for (int idx = tid; idx < D * D; idx += kSegThreads) sm.sref[idx / D][idx % D] = from_f32<T>(a.S_ref[sb + idx]);
  for (int idx = tid; idx < 2 * H * 2 * D; idx += kSegThreads) carry[idx] = 0.f;

  // ---- 3. reverse walk
  BwdPrefetch<T, CH, D> pf;
  if (c_begin < c_end) pf.load(g, a, p, bh, c_end - 1, rw + (size_t)(c_end - 1) * 2 * D * D, tid, lane, wave);
  for (int c = c_end - 1; c >= c_begin; --c) {
    // per-lane indices re-derived every chunk: keeps the compiler from hoisting every per-lane
    // address out of the loop and holding (or spilling) them across the whole walk
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & (kWave - 1), wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int t0 = c * g.Lc, t1 = min(g.T, t0 + g.Lc), L = t1 - t0;
    const bool bufchunk = (c == 0) && g.has_buf;
    const bool clamp_in = (c > 0) && clamp_after(g, t0);
    const bool first = c == c_begin, last = c == c_end - 1;
    const float* Sin_g = rw + (size_t)c * 2 * D * D;   // raw
    const float* Zin_g = Sin_g + (size_t)D * D;
    float* cur_carry = carry + (size_t)(c & 1) * H * 2 * D;        // this chunk's halo -> chunk c-1
    float* prev_carry = carry + (size_t)((c + 1) & 1) * H * 2 * D; // chunk c+1's halo -> this chunk's tail
    __syncthreads();

    // ---- loads: this chunk's inputs (prefetched one chunk ahead) -> LDS; next chunk's prefetch
    {
      pf.store(g, a, sm, tid);
      // carried adjoint (registers) and the saved chunk-start state -> LDS operands, Grams
      float gss = 0.f, gsz = 0.f, gzz = 0.f;
#pragma unroll
      for (int j = 0; j < NT2; ++j) {
        const int tile = wave + kSegWaves * j;
        if (tile >= NTD * NTD) continue;
        const int i0 = (tile / NTD) * 16 + 4 * (lane >> 4), k = (tile % NTD) * 16 + (lane & 15);
        float sv[4], zv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sv[r] = clamp_in ? clamp100(pf.s_in[j][r]) : pf.s_in[j][r];
          zv[r] = g.momentum ? pf.z_in[j][r] : 0.f;
          gss += dS[j][r] * sv[r]; gsz += dS[j][r] * zv[r]; gzz += dZ[j][r] * zv[r];
        }
        // rows i0..i0+3 of column k are contiguous in the transposed copies
        store4<T>(&sm.dSeT[k][i0], dS[j][0], dS[j][1], dS[j][2], dS[j][3]);
        store4<T>(&sm.dZeT[k][i0], dZ[j][0], dZ[j][1], dZ[j][2], dZ[j][3]);
        if constexpr (SIL) {
          store4<T>(&sm.SinT[k][i0], sv[0], sv[1], sv[2], sv[3]);
          store4<T>(&sm.ZinT[k][i0], zv[0], zv[1], zv[2], zv[3]);
        }
      }
      gss = row_sum16(gss); gsz = row_sum16(gsz); gzz = row_sum16(gzz);
      if ((lane & 15) == 0) {
        float* rd = sm.red[wave][lane >> 4];
        rd[0] = gss; rd[1] = gsz; rd[2] = gzz;
      }
      if (c - 1 >= c_begin) pf.load(g, a, p, bh, c - 1, rw + (size_t)(c - 1) * 2 * D * D, tid, lane, wave);
    }
    __syncthreads();
    if (tid < 3) {
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < kSegWaves; ++w)
#pragma unroll
        for (int r = 0; r < 4; ++r) sum += sm.red[w][r][tid];
      sm.gram[tid] = sum;
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

    // ---- phase A: G1 delta^T[s][i] = (S_ref phi_s)[i] - v_s[i] (all waves; the accumulator of lane
    // (i0..i0+3, s) is contiguous in deltaT, so v is read and delta written in place with one
    // 4-element access each). Tile indices past the end are clamped: the MFMAs stay unconditional
    // and only the stores are guarded.
    {
      constexpr int NT1 = NTS * NTD, PER1 = (NT1 + kSegWaves - 1) / kSegWaves;
#pragma unroll 1
      for (int j = 0; j < PER1; ++j) {
        const int tile = min(wave + kSegWaves * j, NT1 - 1);
        const bool valid = NT1 % kSegWaves == 0 || wave + kSegWaves * j < NT1;
        const int m0 = (tile % NTD) * 16, n0 = (tile / NTD) * 16;   // m: rows i, n: sources s
        f32x4 acc = zero4();
#pragma unroll
        for (int k0 = 0; k0 < D; k0 += M::KS)
          acc = M::mma(frag_ld_row<T>(&sm.sref[0][0], D + 8, m0, k0), frag_ld_row<T>(&sm.phi[0][0], D + 8, n0, k0), acc);
        if (valid) {
          const int s = n0 + (lane & 15), i0 = m0 + 4 * (lane >> 4);
          const int pp = t0 - H + s;
          const bool src_ok = s < H + L && pp >= 0;
          float d[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) d[r] = src_ok ? acc[r] - to_f32(sm.deltaT[s][i0 + r]) : 0.f;
          store4<T>(&sm.deltaT[s][i0], d[0], d[1], d[2], d[3]);
        }
      }
    }
    __syncthreads();
    // G2 / G3: Kmat = psi phi^T, K3 = dy delta -> Q^T, Q', Q'^T, Lm
    {
      constexpr int NTQ = NTC * NTS, PERQ = (NTQ + kSegWaves - 1) / kSegWaves;
#pragma unroll 1
      for (int j = 0; j < PERQ; ++j) {
        const int tile = min(wave + kSegWaves * j, NTQ - 1);
        const bool valid = NTQ % kSegWaves == 0 || wave + kSegWaves * j < NTQ;
        const int m0 = (tile / NTS) * 16, n0 = (tile % NTS) * 16;
        f32x4 kk = zero4(), k3 = zero4();
#pragma unroll
        for (int k0 = 0; k0 < D; k0 += M::KS) {
          kk = M::mma(frag_ld_row<T>(&sm.psi[0][0], D + 8, m0, k0), frag_ld_row<T>(&sm.phi[0][0], D + 8, n0, k0), kk);
          k3 = M::mma(frag_ld_row<T>(&sm.dy[0][0], D + 8, m0, k0), frag_ld_row<T>(&sm.deltaT[0][0], D + 8, n0, k0), k3);
        }
        if (valid) {
          const int s = n0 + (lane & 15);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = m0 + 4 * (lane >> 4) + r;
            const float w = to_f32(sm.wsh[t][s]);
            sm.g.QT[s][t] = from_f32<T>(w * kk[r]);
            const T qp = from_f32<T>(w * k3[r]);
            sm.g.Qp[t][s] = qp;
            sm.g.QpT[s][t] = qp;
            sm.Lm[t][s] = kk[r] * k3[r];
          }
        }
      }
    }
    __syncthreads();

    // ---- phase B: G4  dDelta[i, s] = Wz_end[s] (dZ_end phi_s)_i - Ws_end[s] (dS_end phi_s)_i - sum_q dy_q[i] Q[q, s]
    {
      constexpr int NT4 = NTD * NTS, PER4 = (NT4 + kSegWaves - 1) / kSegWaves;
#pragma unroll 1
      for (int j = 0; j < PER4; ++j) {
        const int tile = min(wave + kSegWaves * j, NT4 - 1);
        const bool valid = NT4 % kSegWaves == 0 || wave + kSegWaves * j < NT4;
        const int m0 = (tile / NTS) * 16, n0 = (tile % NTS) * 16;
        f32x4 az = zero4(), as = zero4(), aq = zero4();
#pragma unroll
        for (int k0 = 0; k0 < D; k0 += M::KS) {
          const typename M::frag fb = frag_ld_row<T>(&sm.phi[0][0], D + 8, n0, k0);
          as = M::mma(frag_ld_tr<T>(&sm.dSeT[0][0], D + 8, m0, k0), fb, as);
          az = M::mma(frag_ld_tr<T>(&sm.dZeT[0][0], D + 8, m0, k0), fb, az);
        }
#pragma unroll
        for (int k0 = 0; k0 < CH; k0 += M::KS)
          aq = M::mma(frag_ld_tr<T>(&sm.dy[0][0], D + 8, m0, k0), frag_ld_row<T>(&sm.g.QT[0][0], CH + 8, n0, k0), aq);
        if (valid) {
          const int s = n0 + (lane & 15);
          const float wz = sm.sc.wzend[s], ws = sm.sc.wsend[s];
          float hs = 0.f, hz = 0.f, dd[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = m0 + 4 * (lane >> 4) + r;
            const float d = to_f32(sm.deltaT[s][i]);
            hs += d * as[r];
            hz += d * az[r];
            dd[r] = wz * az[r] - ws * as[r] - aq[r];
          }
          store4<T>(&sm.g.dDT[s][m0 + 4 * (lane >> 4)], dd[0], dd[1], dd[2], dd[3]);
          hs += __shfl_xor(hs, 16); hs += __shfl_xor(hs, 32);
          hz += __shfl_xor(hz, 16); hz += __shfl_xor(hz, 32);
          if (lane < 16) { atomicAdd(&sm.hS[s], hs); atomicAdd(&sm.hZ[s], hz); }
        }
      }
    }
    // G7 (independent of G4) in the same phase
    {   // G7: dpsi[q, k] = a_{q-1} (dy_q S_in)[k] - kappa_{q-1} (dy_q Z_in)[k] - sum_s Q'[q, s] phi_s[k],
        // computed as transposed tiles: a lane holds features k0..k0+3 of one target q
      constexpr int NT7 = NTC * NTD, PER7 = (NT7 + kSegWaves - 1) / kSegWaves;
#pragma unroll 1
      for (int j = 0; j < PER7; ++j) {
        const int tile = min(wave + kSegWaves * j, NT7 - 1);
        const bool valid = NT7 % kSegWaves == 0 || wave + kSegWaves * j < NT7;
        const int m0 = (tile % NTD) * 16, n0 = (tile / NTD) * 16;   // m: features k, n: targets q
        f32x4 as = zero4(), az = zero4(), aq = zero4();
#pragma unroll
        for (int k0 = 0; k0 < D; k0 += M::KS) {
          const typename M::frag fb = frag_ld_row<T>(&sm.dy[0][0], D + 8, n0, k0);
          if constexpr (SIL) {
            as = M::mma(frag_ld_row<T>(&sm.SinT[0][0], D + 8, m0, k0), fb, as);
            az = M::mma(frag_ld_row<T>(&sm.ZinT[0][0], D + 8, m0, k0), fb, az);
          } else {   // S_in[i][k] straight from the saved fp32 state (16 consecutive k per row i)
            typename M::frag fs;
            {
              const int kb = k0 + (lane >> 4) * M::KL;
              const float* q = Sin_g + (size_t)kb * D + m0 + (lane & 15);
              if constexpr (M::KL == 1) fs = static_cast<T>(clamp_in ? clamp100(q[0]) : q[0]);
              else {
#pragma unroll
                for (int ee = 0; ee < M::KL; ++ee) {
                  const float x = q[(size_t)ee * D];
                  fs[ee] = static_cast<T>(clamp_in ? clamp100(x) : x);
                }
              }
            }
            as = M::mma(fs, fb, as);
            az = M::mma(frag_ld_or_zero<T>(g.momentum ? Zin_g : nullptr, 1, D, m0, k0), fb, az);
          }
        }
#pragma unroll
        for (int k0 = 0; k0 < SPM; k0 += M::KS)
          aq = M::mma(frag_ld_tr<T>(&sm.phi[0][0], D + 8, m0, k0), frag_ld_row<T>(&sm.g.Qp[0][0], SPM + 8, n0, k0), aq);
        const int t = n0 + (lane & 15), kq = m0 + 4 * (lane >> 4);
        const float ac = sm.sc.acoef[t], kc = sm.sc.kcoef[t];
        float ps[4], dpsi[4], fsp = 0.f, fzp = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          ps[r] = to_f32(sm.psi[t][kq + r]);
          dpsi[r] = ac * as[r] - kc * az[r] - aq[r];
          fsp += as[r] * ps[r];
          fzp += az[r] * ps[r];
        }
        if (bufchunk) {
          for (int s = 0; s < H; ++s) {
            const float* Bs = a.buf_in + ((size_t)bh * H + s) * D * D;
            f32x4 ab = zero4();
#pragma unroll
            for (int k0 = 0; k0 < D; k0 += M::KS)
              ab = M::mma(frag_ld<T>(Bs, 1, D, m0, k0), frag_ld_row<T>(&sm.dy[0][0], D + 8, n0, k0), ab);
            const float w = to_f32(sm.wsh[t][s]);
            float lm = 0.f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              dpsi[r] -= w * ab[r];
              lm += ab[r] * ps[r];
            }
            lm += __shfl_xor(lm, 16);
            lm += __shfl_xor(lm, 32);
            if (valid && lane < 16) atomicAdd(&sm.Lm[t][s], lm);
          }
        }
        fsp += __shfl_xor(fsp, 16); fsp += __shfl_xor(fsp, 32);
        fzp += __shfl_xor(fzp, 16); fzp += __shfl_xor(fzp, 32);
        if (valid) {
          if (lane < 16) { atomicAdd(&sm.fS[t], fsp); atomicAdd(&sm.fZ[t], fzp); }
          if (t < L) {
            const size_t row = (tb + t0 + t) * D + kq;
            if (g.map_mode == MAP_ELEMENTWISE) {
#pragma unroll
              for (int r = 0; r < 4; ++r) dpsi[r] *= poly_map_grad(to_f32(a.q[row + r]), g.map_deg);
            }
            store4<T>(a.dq + row, dpsi[0], dpsi[1], dpsi[2], dpsi[3]);
          }
        }
      }
    }
    __syncthreads();

    // ---- phase C: dv from dDelta; G6 dS_ref; d buffer_in; then G5 and the carried adjoint (no barrier between)
    {   // dv: 8 features of one source per lane
      const int tail0 = t1 - H;
      constexpr int NV = D / 8;
      for (int idx = tid; idx < (H + L) * NV; idx += kSegThreads) {
        const int s = idx / NV, i0 = (idx % NV) * 8;
        const int pp = t0 - H + s;
        if (pp < 0) continue;
        const Vec8<T> x = vec8_load(&sm.g.dDT[s][i0]);
        float val[8];
#pragma unroll
        for (int e8 = 0; e8 < 8; ++e8) val[e8] = -to_f32(x.v[e8]);
        if (s < H) {
          float* dst = first ? (c > 0 ? p.halo_part + (((size_t)bh * sg.nseg + seg) * H + s) * (2 * D) + i0 : nullptr)
                             : cur_carry + s * 2 * D + i0;
          if (dst) store8f(dst, val);
          continue;
        }
        if (pp >= tail0) add8f(val, prev_carry + (pp - tail0) * 2 * D + i0);
        if (pp >= seg_tail0) {
          store8f(p.tail_part + (((size_t)bh * sg.nseg + seg) * H + (pp - seg_tail0)) * (2 * D) + i0, val);
        } else {
          Vec8<T> y;
#pragma unroll
          for (int e8 = 0; e8 < 8; ++e8) y.v[e8] = from_f32<T>(val[e8]);
          y.store(a.dv + (tb + pp) * D + i0);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < NT2; ++j) {   // G6: dS_ref[i, k] += sum_s dDelta[i, s] phi_s[k]
      const int tile = min(wave + kSegWaves * j, NTD * NTD - 1);
      const int m0 = (tile / NTD) * 16, n0 = (tile % NTD) * 16;
      f32x4 acc = zero4();
#pragma unroll
      for (int k0 = 0; k0 < SPM; k0 += M::KS)
        acc = M::mma(frag_ld_tr<T>(&sm.g.dDT[0][0], D + 8, m0, k0), frag_ld_tr<T>(&sm.phi[0][0], D + 8, n0, k0), acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) dsr[j][r] += acc[r];
    }
    if (bufchunk) {   // d buffer_in[s] = Wz_end[s] dZ_end - Ws_end[s] dS_end - sum_q Ws[s, q-1] dy_q psi_q^T
      for (int s = 0; s < H; ++s) {
        float* dst = a.dbuf_in + ((size_t)bh * H + s) * D * D;
#pragma unroll
        for (int j = 0; j < NT2; ++j) {
          const int tile = min(wave + kSegWaves * j, NTD * NTD - 1);
          const bool valid = (NTD * NTD) % kSegWaves == 0 || wave + kSegWaves * j < NTD * NTD;
          const int m0 = (tile / NTD) * 16, n0 = (tile % NTD) * 16;
          f32x4 acc = zero4();
#pragma unroll
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
            acc = M::mma(fa, frag_ld_tr<T>(&sm.psi[0][0], D + 8, n0, k0), acc);
          }
          if (valid) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int i = m0 + 4 * (lane >> 4) + r, k = n0 + (lane & 15);
              dst[(size_t)i * D + k] = sm.sc.wzend[s] * dZ[j][r] - sm.sc.wsend[s] * dS[j][r] - acc[r];
            }
          }
        }
      }
    }
    // ---- phase D: G5  dphi[s, k] = Wz_end dZ_end^T delta_s - Ws_end dS_end^T delta_s - sum_q Q'[q, s] psi_q + S_ref^T dDelta_s,
    // as transposed tiles: a lane holds features k0..k0+3 of one source s
    {
      const int tail0 = t1 - H;
      constexpr int NT5 = NTS * NTD, PER5 = (NT5 + kSegWaves - 1) / kSegWaves;
#pragma unroll 1
      for (int j = 0; j < PER5; ++j) {
        const int tile = min(wave + kSegWaves * j, NT5 - 1);
        const bool valid = NT5 % kSegWaves == 0 || wave + kSegWaves * j < NT5;
        const int m0 = (tile % NTD) * 16, n0 = (tile / NTD) * 16;   // m: features k, n: sources s
        f32x4 a1 = zero4(), a2 = zero4(), a3 = zero4(), a4 = zero4();
#pragma unroll
        for (int k0 = 0; k0 < D; k0 += M::KS) {
          const typename M::frag fb = frag_ld_row<T>(&sm.deltaT[0][0], D + 8, n0, k0);
          a1 = M::mma(frag_ld_row<T>(&sm.dZeT[0][0], D + 8, m0, k0), fb, a1);
          a2 = M::mma(frag_ld_row<T>(&sm.dSeT[0][0], D + 8, m0, k0), fb, a2);
          a4 = M::mma(frag_ld_tr<T>(&sm.sref[0][0], D + 8, m0, k0), frag_ld_row<T>(&sm.g.dDT[0][0], D + 8, n0, k0), a4);
        }
#pragma unroll
        for (int k0 = 0; k0 < CH; k0 += M::KS)
          a3 = M::mma(frag_ld_tr<T>(&sm.psi[0][0], D + 8, m0, k0), frag_ld_row<T>(&sm.g.QpT[0][0], CH + 8, n0, k0), a3);
        const int s = n0 + (lane & 15), kq = m0 + 4 * (lane >> 4);
        const int pp = t0 - H + s;
        if (valid && s < H + L && pp >= 0) {
          const float wz = sm.sc.wzend[s], ws = sm.sc.wsend[s];
          float val[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) val[r] = wz * a1[r] - ws * a2[r] - a3[r] + a4[r];
          if (s < H) {
            float* dst = first ? (c > 0 ? p.halo_part + (((size_t)bh * sg.nseg + seg) * H + s) * (2 * D) + D + kq : nullptr)
                               : cur_carry + s * 2 * D + D + kq;
            if (dst) store4<float>(dst, val[0], val[1], val[2], val[3]);
          } else {
            if (pp >= tail0) {
              const float4 cv = *reinterpret_cast<const float4*>(prev_carry + (pp - tail0) * 2 * D + D + kq);
              val[0] += cv.x; val[1] += cv.y; val[2] += cv.z; val[3] += cv.w;
            }
            if (pp >= seg_tail0) {
              store4<float>(p.tail_part + (((size_t)bh * sg.nseg + seg) * H + (pp - seg_tail0)) * (2 * D) + D + kq,
                            val[0], val[1], val[2], val[3]);
            } else {
              const size_t row = (tb + pp) * D + kq;
              if (g.map_mode == MAP_ELEMENTWISE) {
#pragma unroll
                for (int r = 0; r < 4; ++r) val[r] *= poly_map_grad(to_f32(a.k[row + r]), g.map_deg);
              }
              store4<T>(a.dk + row, val[0], val[1], val[2], val[3]);
            }
          }
        }
      }
    }

    // ---- phase E: chunk-start adjoint (the transposed chunk transition) -> carried (dS, dZ) for chunk c - 1
    {
      const float ae = sm.sc.endc[0], ke = sm.sc.endc[1], be = sm.sc.endc[2];
#pragma unroll
      for (int j = 0; j < NT2; ++j) {
        const int tile = min(wave + kSegWaves * j, NTD * NTD - 1);
        const bool valid = (NTD * NTD) % kSegWaves == 0 || wave + kSegWaves * j < NTD * NTD;
        const int m0 = (tile / NTD) * 16, n0 = (tile % NTD) * 16;
        f32x4 aa = zero4(), ak = zero4();
#pragma unroll
        for (int k0 = 0; k0 < CH; k0 += M::KS) {
          const typename M::frag fb = frag_ld_tr<T>(&sm.psi[0][0], D + 8, n0, k0);
          aa = M::mma(frag_ld_tr_kscaled<T>(&sm.dy[0][0], D + 8, m0, k0, sm.sc.acoef), fb, aa);
          ak = M::mma(frag_ld_tr_kscaled<T>(&sm.dy[0][0], D + 8, m0, k0, sm.sc.kcoef), fb, ak);
        }
        if (valid) {
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
    }

    // ---- inputs of the scalar gradients (k_bwd_scalar) -> HBM
    __syncthreads();   // hS, hZ, fS, fZ, Lm complete
    {
      typedef ScalarBlock<CH> SB;
      float* blk = p.scal + ((size_t)bh * g.nc + c) * SB::SIZE;
      for (int idx = tid; idx < CH * SPM; idx += kSegThreads) blk[SB::LM + idx] = sm.Lm[idx / SPM][idx % SPM];
      for (int idx = tid; idx < SPM; idx += kSegThreads) { blk[SB::HS + idx] = sm.hS[idx]; blk[SB::HZ + idx] = sm.hZ[idx]; }
      if (tid < CH) { blk[SB::FS + tid] = sm.fS[tid]; blk[SB::FZ + tid] = sm.fZ[tid]; }
      if (tid < 4) blk[SB::GRAM + tid] = tid < 3 ? sm.gram[tid] : 0.f;
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
// adjoint at every segment end: grid (D * D / kThreads, BH)
//   x_{j-1} = [[a_j, 0], [-kappa_j, b_j]] x_j + [L_j; K_j], starting from (dS_T * clamp mask, dZ_T)
// ---------------------------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(kThreads) void k_bwd_seg_scan(const Geom g, const float* dS_T, const float* dZ_T,
                                                             const SegGeom sg, const BwdSegPtrs p) {
  if (geom_skip(g)) return;
  const int bh = blockIdx.y;
  const int idx = blockIdx.x * kThreads + threadIdx.x;
  if (idx >= D * D) return;
  const size_t off = (size_t)bh * D * D + idx;
  float dS = dS_T ? dS_T[off] : 0.f;
  if (g.clamp_final) dS *= clamp_mask(p.final_raw[off]);
  float dZ = (g.momentum && dZ_T) ? dZ_T[off] : 0.f;
  const float* ag = p.adj_agg + (size_t)bh * sg.nseg * sg.agg_stride;
  float* sa = p.seg_adj + (size_t)bh * sg.nseg * 2 * D * D;
  // aggregates are read kScanBatch segments at a time (one memory round trip per batch)
  for (int j0 = sg.nseg - 1; j0 >= 0; j0 -= kScanBatch) {
    float Lv[kScanBatch], Kv[kScanBatch], ta[kScanBatch], tk[kScanBatch], tbb[kScanBatch];
#pragma unroll
    for (int u = 0; u < kScanBatch; ++u) {
      const float* aj = ag + (size_t)max(j0 - u, 0) * sg.agg_stride;
      Lv[u] = aj[idx]; Kv[u] = aj[D * D + idx];
      ta[u] = aj[2 * D * D]; tk[u] = aj[2 * D * D + 1]; tbb[u] = aj[2 * D * D + 2];
    }
#pragma unroll
    for (int u = 0; u < kScanBatch; ++u) {
      const int js = j0 - u;
      if (js >= 0) {
        sa[(size_t)js * 2 * D * D + idx] = dS;
        sa[(size_t)js * 2 * D * D + D * D + idx] = dZ;
        const float s_out = dS;
        dS = ta[u] * s_out + Lv[u];
        dZ = g.momentum ? (tbb[u] * dZ - tk[u] * s_out + Kv[u]) : 0.f;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// segment-boundary fixup: grid (nseg, BH)
// ---------------------------------------------------------------------------------------------
// reduce_dsref: without d buffer_out terms (which add to the dS_ref partials here) the block of
// segment seg also sums its share of the dS_ref partials over the segments (no separate launch).
template <typename T, int D>
__global__ __launch_bounds__(kThreads) void k_bwd_seg_fixup(const Geom g, const BwdPtrs<T> a, const SegGeom sg,
                                                              const BwdSegPtrs p, int reduce_dsref) {
  if (geom_skip(g)) return;
  if (a.dbuf_out) bwd_seg_fixup<T, D, true>(g, a, sg, p, reduce_dsref, blockIdx.x, blockIdx.y);
  else bwd_seg_fixup<T, D, false>(g, a, sg, p, reduce_dsref, blockIdx.x, blockIdx.y);
}

// dS_ref = sum over segments of the partials.   grid (D*D/256, BH)
__global__ __launch_bounds__(kThreads) void k_seg_reduce_dsref(const Geom g, int nseg, int n, const float* part,
                                                                float* out) {
  if (geom_skip(g)) return;
  const int bh = blockIdx.y;
  const int idx = blockIdx.x * kThreads + threadIdx.x;
  if (idx >= n) return;
  float acc = 0.f;
  for (int s = 0; s < nseg; ++s) acc += part[((size_t)bh * nseg + s) * n + idx];
  out[(size_t)bh * n + idx] = acc;
}

template <typename T, int CH, int D>
size_t bwd_seg_smem_bytes(int H) {
  return carry_offset<BwdSegSmem<T, CH, D>>() + (size_t)2 * H * 2 * D * sizeof(float);
}

hipError_t launch_walk_bwd_kernel(const Geom& g, const BwdPtrs<bf16>& a, const SegGeom& sg, const BwdSegPtrs& p,
                                  hipStream_t stream);
hipError_t launch_scalar_chain(const Geom& g, const BwdPtrs<bf16>& a, const BwdSegPtrs& p, const SegGeom& sg,
                               bool with_fixup, hipStream_t stream);
hipError_t launch_buf_bwd(const Geom& g, const BwdPtrs<bf16>& a, const BwdSegPtrs& p, hipStream_t stream);
hipError_t launch_chunk_bwd(const Geom& g, const BwdPtrs<bf16>& a, const SegGeom& sg, const BwdSegPtrs& p,
                            hipStream_t stream);

// walk: run the specialised reverse walk (walk_bwd.hip, bf16 with d = 64 only) in place of k_bwd_seg
// ag (the specialised path): adjoint aggregates over the forward's chunks (seg_common.h).
template <typename T, int CH, int D>
hipError_t launch_bwd_seg(const Geom& g, const BwdPtrs<T>& a, const SegGeom& sg, const BwdSegPtrs& p,
                          hipStream_t stream, bool walk, const AggOverFwd* ag) {
  // the chunk coefficient records p.coef / p.wsh were formed by the forward (input-only)
  hipError_t err = hipSuccess;
  if (sg.nseg > 1) {
    if constexpr (sizeof(T) == 2 && CH == 32 && D == 64) {
      if (ag) {
        if (ag->sg.nseg != sg.nseg || ag->sg.agg_stride != sg.agg_stride) return hipErrorInvalidValue;
        BwdSegPtrs pf = p;
        pf.coef = const_cast<float*>(ag->coef);
        const size_t smem = sizeof(BwdAggSmem<T, 64, D>);
        err = set_dyn_smem(reinterpret_cast<const void*>(&k_bwd_seg_agg<T, 64, D>), smem);
        if (err != hipSuccess) return err;
        prof_begin(KID_BWD_ADJOINT, stream);
        hipLaunchKernelGGL((k_bwd_seg_agg<T, 64, D>), dim3(sg.nseg, g.BH), dim3(kSegThreads), smem, stream, ag->g, a,
                           ag->sg, pf);
        prof_end(KID_BWD_ADJOINT, stream);
        if ((err = hipGetLastError()) != hipSuccess) return err;
      }
    }
    if (!ag) {
      const size_t smem = sizeof(BwdAggSmem<T, CH, D>);
      err = set_dyn_smem(reinterpret_cast<const void*>(&k_bwd_seg_agg<T, CH, D>), smem);
      if (err != hipSuccess) return err;
      prof_begin(KID_BWD_ADJOINT, stream);
      hipLaunchKernelGGL((k_bwd_seg_agg<T, CH, D>), dim3(sg.nseg, g.BH), dim3(kSegThreads), smem, stream, g, a, sg, p);
      prof_end(KID_BWD_ADJOINT, stream);
      if ((err = hipGetLastError()) != hipSuccess) return err;
    }
  }
  prof_begin(KID_BWD_SCAN, stream);
  hipLaunchKernelGGL((k_bwd_seg_scan<D>), dim3((D * D + kThreads - 1) / kThreads, g.BH), dim3(kThreads), 0, stream,
                     g, a.dS_T, a.dZ_T, sg, p);
  prof_end(KID_BWD_SCAN, stream);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  if constexpr (sizeof(T) == 2 && CH == 32 && D == 64) {
    if (ag && ag->chunk_bwd) return launch_chunk_bwd(ag->g, a, ag->sg, p, stream);
    if (walk) {
      prof_name(KID_BWD_CHUNK, "k_walk_bwd");
      prof_begin(KID_BWD_CHUNK, stream);
      err = launch_walk_bwd_kernel(g, a, sg, p, stream);
      prof_end(KID_BWD_CHUNK, stream);
      if (err != hipSuccess) return err;
      // a carried buffer: its first-chunk terms, before the scalar chain reads chunk 0's record
      if (p.buf_adj && (err = launch_buf_bwd(g, a, p, stream)) != hipSuccess) return err;
    }
  }
  if (!walk) {
    const size_t smem = bwd_seg_smem_bytes<T, CH, D>(g.H);
    err = set_dyn_smem(reinterpret_cast<const void*>(&k_bwd_seg<T, CH, D>), smem);
    if (err != hipSuccess) return err;
    prof_name(KID_BWD_CHUNK, "k_bwd_seg");
    prof_begin(KID_BWD_CHUNK, stream);
    hipLaunchKernelGGL((k_bwd_seg<T, CH, D>), dim3(sg.nseg, g.BH), dim3(kSegThreads), smem, stream, g, a, sg, p);
    prof_end(KID_BWD_CHUNK, stream);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  // the specialised path runs the fixup inside the scalar-chain launch when the two are independent
  // (no token gates, whose gradients the fixup forms from the chains' output; no buffer_out gradient)
  const int fused_reduce = a.dbuf_out == nullptr;
  const bool fixup_in_chain = walk && fused_reduce && g.gate_mode != GATE_TOKEN;
  if constexpr (sizeof(T) == 2 && CH == 32 && D == 64) {
    if (walk) {
      prof_name(KID_BWD_SCALAR, fixup_in_chain ? "k_scalar_chain+fixup" : "k_scalar_chain");
      prof_begin(KID_BWD_SCALAR, stream);
      err = launch_scalar_chain(g, a, p, sg, fixup_in_chain, stream);
      prof_end(KID_BWD_SCALAR, stream);
      if (err != hipSuccess) return err;
    }
  }
  if (!walk && (err = launch_bwd_scalar<T, CH>(g, a, p, stream)) != hipSuccess) return err;
  if (fixup_in_chain) return hipSuccess;
  prof_begin(KID_BWD_FIXUP, stream);
  hipLaunchKernelGGL((k_bwd_seg_fixup<T, D>), dim3(sg.nseg, g.BH), dim3(kThreads), 0, stream, g, a, sg, p,
                     fused_reduce);
  prof_end(KID_BWD_FIXUP, stream);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  if (fused_reduce) return hipSuccess;
  prof_begin(KID_REDUCE_DSREF, stream);
  hipLaunchKernelGGL(k_seg_reduce_dsref, dim3((D * D + kThreads - 1) / kThreads, g.BH), dim3(kThreads), 0, stream,
                     g, sg.nseg, D * D, (const float*)p.dsref_part, a.dS_ref);
  prof_end(KID_REDUCE_DSREF, stream);
  return hipGetLastError();
}

#define ATLAS_INST_BWD_SEG(T, CH, D)                                                                  \
  template hipError_t launch_bwd_seg<T, CH, D>(const Geom&, const BwdPtrs<T>&, const SegGeom&,        \
                                               const BwdSegPtrs&, hipStream_t, bool, const AggOverFwd*); \
  template size_t bwd_seg_smem_bytes<T, CH, D>(int);

ATLAS_INST_BWD_SEG(bf16, 32, 64)
ATLAS_INST_BWD_SEG(float, 16, 64)
ATLAS_INST_BWD_SEG(bf16, 32, 32)
ATLAS_INST_BWD_SEG(float, 16, 32)

}  // namespace atlas
