// seg_fwd.h - the segment walk of the forward recurrence (aggregate pass and full walk).
//
// Every chunk is a handful of small GEMMs separated by workgroup barriers; with 8 waves per CU the
// barriers and LDS latency, not the matrix cores, set the pace. All tile counts and k extents are
// therefore compile-time (the source tile always spans SPM = CH + 32 rows, padded rows are zero)
// so that each wave's fragment loads are issued together ahead of its MFMA chains.
#pragma once

#include "mem_common.h"
#include "mem_params.h"
#include "seg_common.h"

namespace atlas {

template <typename T, int CH, int D, bool FULL>
struct SegFwdSmem {
  static constexpr int SPM = CH + kHaloPad;
  alignas(16) T phi[SPM][D + 8];   // phi[s][k]
  alignas(16) T vd[SPM][D + 8];    // v[s][i] staged by the loads, then delta[s][i]
  alignas(16) T sref[D][D + 8];
  ChunkScalars<CH> sc;
  // full walk only
  T psi[FULL ? CH : 1][D + 8];
  T Q[FULL ? CH : 1][SPM + 8];
  T Sb[FULL ? D : 1][D + 8];
  T Zb[FULL ? D : 1][D + 8];
  T wsh[FULL ? CH : 1][SPM + 8];       // Ws[s, tau-1]
};

// Per-thread register prefetch of one chunk's inputs (issued one chunk ahead).
// Every load is unconditional from an in-bounds address (out-of-range rows are redirected to the
// chunk's first token, absent optional inputs to `decay`); the raw values are kept with validity
// flags and only converted and masked in store(). A load under a condition whose value is
// converted inside the same branch would make the wave wait for each load in turn.
template <typename T, int CH, int D, bool FULL>
struct ChunkPrefetch {
  static constexpr int SPM = CH + kHaloPad;
  static constexpr int NV_PHI = (SPM * D / 8 + kSegThreads - 1) / kSegThreads;
  static constexpr int NV_PSI = FULL ? (CH * D / 8 + kSegThreads - 1) / kSegThreads : 0;
  static constexpr int NWL = (CH * kMaxWindow + kSegThreads - 1) / kSegThreads;
  static constexpr int REC4 = CoefRec<CH>::SIZE / 4;
  static constexpr int NV_WSH = FULL ? (CH * SPM / 8 + kSegThreads - 1) / kSegThreads : 0;
  static_assert(REC4 <= kSegThreads && SPM % 8 == 0, "record / wsh prefetch");
  Vec8<T> phi[NV_PHI];
  Vec8<T> vv[NV_PHI];
  Vec8<T> psi[NV_PSI > 0 ? NV_PSI : 1];
  Vec8<T> wsv[NV_WSH > 0 ? NV_WSH : 1];
  float rc0, rc1, rc2, rc3;   // this thread's float4 of the coefficient record
  T alpha, eta, beta, ug;
  T wl[NWL];
  unsigned ok_phi, ok_psi, ok_wl;
  bool ok_t, ok_ug, pad_ug;

  // rec_c / wsh_c: this chunk's coefficient record and Ws[s, t-1] block (k_chunk_coef)
  __device__ __forceinline__ void load(const Geom& g, const FwdPtrs<T>& a, size_t tb, int t0, int L,
                                       const float* rec_c, const T* wsh_c) {
    const int tid = threadIdx.x, H = g.H;
    const size_t r0 = tb + t0;                          // always a valid token row
    ok_phi = 0; ok_psi = 0; ok_wl = 0;
    {
      const float4 r4 = reinterpret_cast<const float4*>(rec_c)[tid < REC4 ? tid : 0];
      rc0 = r4.x; rc1 = r4.y; rc2 = r4.z; rc3 = r4.w;
    }
    if constexpr (FULL) {
#pragma unroll
      for (int j = 0; j < NV_WSH; ++j) {
        const int v = tid + j * kSegThreads;
        wsv[j] = vec8_load(wsh_c + (size_t)(v < CH * SPM / 8 ? v : 0) * 8);
      }
    }
#pragma unroll
    for (int j = 0; j < NV_PHI; ++j) {
      const int v = tid + j * kSegThreads;
      {   // phi and v: 8 consecutive features of source s per lane
        const int s = v / (D / 8), c8 = v % (D / 8);
        const int p = t0 - H + s;
        const bool ok = s < SPM && s < H + L && p >= 0;
        const size_t off = (ok ? tb + p : r0) * D + c8 * 8;
        phi[j] = vec8_load(a.k + off);
        vv[j] = vec8_load(a.v + off);
        ok_phi |= (ok ? 1u : 0u) << j;
      }
    }
    if constexpr (FULL) {
#pragma unroll
      for (int j = 0; j < NV_PSI; ++j) {
        const int v = tid + j * kSegThreads;
        const int t = v / (D / 8), c8 = v % (D / 8);
        const bool ok = t < L;
        psi[j] = vec8_load(a.q + (ok ? r0 + t : r0) * D + c8 * 8);
        ok_psi |= (ok ? 1u : 0u) << j;
      }
    }
    ok_t = tid < L;
    const size_t rt = ok_t ? r0 + tid : r0;
    alpha = a.decay[rt];
    eta = a.lr[rt];
    const T* bp = (g.momentum && a.beta) ? a.beta : a.decay;
    beta = bp[rt];
    const T* gp = a.gate ? a.gate : a.decay;
    {
      const int p = t0 - H + tid;
      ok_ug = g.gate_mode == GATE_TOKEN && tid < SPM && tid < H + L && p >= 0;
      pad_ug = g.gate_mode == GATE_TOKEN && tid < SPM && tid < H + L && p < 0;
      ug = gp[ok_ug ? tb + p : r0];
    }
#pragma unroll
    for (int j = 0; j < NWL; ++j) {
      const int idx = tid + j * kSegThreads;
      const bool ok = g.gate_mode == GATE_LAG && idx < CH * g.e && idx / g.e < L;
      wl[j] = gp[ok ? r0 * g.e + idx : r0];
      ok_wl |= (ok ? 1u : 0u) << j;
    }
  }

  template <typename Sm>
  __device__ __forceinline__ void store(const Geom& g, Sm& sm) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < NV_PHI; ++j) {
      const int v = tid + j * kSegThreads;
      const int s = v / (D / 8), c8 = v % (D / 8);
      if (s < SPM) {
        const bool ok = (ok_phi >> j) & 1u;
        Vec8<T> x = phi[j].masked(ok);
        if (g.map_mode == MAP_ELEMENTWISE) x = x.mapped(g.map_deg);
        x.store(&sm.phi[s][c8 * 8]);
        vv[j].masked(ok).store(&sm.vd[s][c8 * 8]);
      }
    }
    if constexpr (FULL) {
#pragma unroll
      for (int j = 0; j < NV_PSI; ++j) {
        const int v = tid + j * kSegThreads;
        const int t = v / (D / 8), c8 = v % (D / 8);
        if (t < CH) {
          Vec8<T> x = psi[j].masked((ok_psi >> j) & 1u);
          if (g.map_mode == MAP_ELEMENTWISE) x = x.mapped(g.map_deg);
          x.store(&sm.psi[t][c8 * 8]);
        }
      }
    }
    if (tid < REC4) reinterpret_cast<float4*>(&sm.sc.acoef[0])[tid] = make_float4(rc0, rc1, rc2, rc3);
    if constexpr (FULL) {
#pragma unroll
      for (int j = 0; j < NV_WSH; ++j) {
        const int v = tid + j * kSegThreads;
        if (v < CH * SPM / 8) wsv[j].store(&sm.wsh[(v * 8) / SPM][(v * 8) % SPM]);
      }
    }
    if (tid < CH) {
      sm.sc.alpha[tid] = ok_t ? to_f32(alpha) : 1.f;
      sm.sc.eta[tid] = ok_t ? to_f32(eta) : 0.f;
      sm.sc.beta[tid] = ok_t ? (g.momentum ? to_f32(beta) : 0.f) : 1.f;
    }
    if (g.gate_mode == GATE_TOKEN && tid < SPM) sm.sc.ug[tid] = ok_ug ? to_f32(ug) : (pad_ug ? 1.f : 0.f);
    if (g.gate_mode == GATE_LAG) {
#pragma unroll
      for (int j = 0; j < NWL; ++j) {
        const int idx = tid + j * kSegThreads;
        if (idx < CH * g.e) sm.sc.wl[idx] = ((ok_wl >> j) & 1u) ? to_f32(wl[j]) : 0.f;
      }
    }
  }
};

enum WalkMode { WALK_AGG = 0, WALK_FULL = 1 };

// Segment walk.
//   WALK_AGG:    zero initial state; writes the segment aggregate (a, kappa, b, U, V) to agg.
//   WALK_FULL:   starts from seg_states[seg] (the segment scan folded the preceding aggregates),
//                walks the chunks with the true state and writes y (and S_T, Z_T, the raw S_{T-1}),
//                and the raw state at every backward-chunk boundary to rw ([BH][ncb][2][D][D]):
//                the chunk start and, when g.Lmid > 0, the state after token Lmid - 1.
// The chunk coefficients (a, kappa, end weights, Ws[s, t-1]) come precomputed from k_chunk_coef
// (coef: [BH][nc] records, wsh_all: [BH][nc][CH][SPM], full walk only) with the prefetch.
// Wave roles per chunk: P1 all waves run G1 (and G2 for the full walk); P3 all waves run G3 (y,
// full walk), then G4 on the state tiles they own, updating the states, which they hold in
// registers.
template <typename T, int CH, int D, int MODE>
__device__ __forceinline__ void fwd_segment(const Geom& g, const FwdPtrs<T>& a, const SegGeom& sg, float* agg,
                                            const float* seg_states, float* rw, float* final_raw,
                                            const float* coef, const T* wsh_all, unsigned char* smem_raw) {
  constexpr bool AGG = MODE == WALK_AGG;
  constexpr bool FULL = MODE == WALK_FULL;
  typedef SegFwdSmem<T, CH, D, FULL> Sm;
  Sm& sm = *reinterpret_cast<Sm*>(smem_raw);
  constexpr int SPM = Sm::SPM;
  constexpr int NTD = D / 16;                    // 16-wide tiles along D
  constexpr int NTS = SPM / 16;                  // 16-wide tiles along the sources
  typedef MM<T> M;
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int seg = blockIdx.x, bh = blockIdx.y;
  const int H = g.H;
  const size_t tb = (size_t)bh * g.T;
  const size_t sb = (size_t)bh * D * D;
  const int c_begin = seg * sg.G, c_end = min(g.nc, c_begin + sg.G);

  // ---- S_ref (bf16/fp32 operand copy)
  for (int idx = tid; idx < D * D; idx += kSegThreads) sm.sref[idx / D][idx % D] = from_f32<T>(a.S_ref[sb + idx]);

  // ---- state registers: the NTD x NTD state tiles are spread over the waves, NOWN tiles of one
  // row tile per wave.
  constexpr int NOWN = NTD * NTD < kSegWaves ? 1 : NTD * NTD / kSegWaves;
  constexpr int OWNERS = NTD * NTD / NOWN;
  static_assert(NTD % NOWN == 0, "owned tiles share a row tile");
  const bool owns = wave < OWNERS;
  const int otile0 = wave * NOWN;                             // first owned tile, row-major over (mt, n)
  const int mt = otile0 / NTD, nt0 = otile0 % NTD;           // row tile, first column tile
  float Sr[NOWN][4], Zr[NOWN][4];
#pragma unroll
  for (int jn = 0; jn < NOWN; ++jn)
#pragma unroll
    for (int r = 0; r < 4; ++r) { Sr[jn][r] = 0.f; Zr[jn][r] = 0.f; }
  float seg_a = 1.f, seg_k = 0.f, seg_b = 1.f;   // aggregate transition (AGG)

  if constexpr (!AGG) {
    // segment-start state (written by the segment scan)
    if (owns) {
      const float* ss = seg_states + ((size_t)bh * sg.nseg + seg) * 2 * D * D;
#pragma unroll
      for (int jn = 0; jn < NOWN; ++jn)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = mt * 16 + 4 * (lane >> 4) + r, k = (nt0 + jn) * 16 + (lane & 15);
          Sr[jn][r] = ss[(size_t)i * D + k];
          Zr[jn][r] = ss[(size_t)D * D + (size_t)i * D + k];
          if constexpr (FULL) {
            sm.Sb[i][k] = from_f32<T>(Sr[jn][r]);
            sm.Zb[i][k] = from_f32<T>(Zr[jn][r]);
          }
        }
    }
  }

  constexpr int REC = CoefRec<CH>::SIZE;
  const float* coef_row = coef + (size_t)bh * g.nc * REC;
  const T* wsh_row = FULL ? wsh_all + (size_t)bh * g.nc * CH * SPM : nullptr;
  ChunkPrefetch<T, CH, D, FULL> pf;
  if (c_begin < c_end) {
    const int t0 = c_begin * g.Lc;
    pf.load(g, a, tb, t0, min(g.T, t0 + g.Lc) - t0, coef_row + (size_t)c_begin * REC,
            FULL ? wsh_row + (size_t)c_begin * CH * SPM : nullptr);
  }

  for (int c = c_begin; c < c_end; ++c) {
    // per-lane indices re-derived every chunk: keeps the compiler from hoisting every per-lane
    // address out of the loop and holding (or spilling) them across the whole walk
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & (kWave - 1), wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int t0 = c * g.Lc;
    const int t1 = min(g.T, t0 + g.Lc);
    const int L = t1 - t0;
    const bool bufchunk = (c == 0) && g.has_buf;
    const int rb = g.Lmid > 0 ? 2 : 1;        // backward chunks per forward chunk
    if constexpr (FULL) {
      // the segment's start state (later chunk starts are written as the previous chunk ends)
      if (owns && c == c_begin) {
        float* dst = rw + ((size_t)bh * g.ncb + (size_t)c * rb) * 2 * D * D;
#pragma unroll
        for (int jn = 0; jn < NOWN; ++jn)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = mt * 16 + 4 * (lane >> 4) + r, k = (nt0 + jn) * 16 + (lane & 15);
            dst[(size_t)i * D + k] = Sr[jn][r];
            dst[(size_t)D * D + (size_t)i * D + k] = Zr[jn][r];
          }
      }
    }
    __syncthreads();                      // previous chunk finished with the LDS inputs
    pf.store(g, sm);
    __syncthreads();
    if (c + 1 < c_end) {                  // prefetch the next chunk while this one computes
      const int n0 = (c + 1) * g.Lc;
      pf.load(g, a, tb, n0, min(g.T, n0 + g.Lc) - n0, coef_row + (size_t)(c + 1) * REC,
              FULL ? wsh_row + (size_t)(c + 1) * CH * SPM : nullptr);
    }

    // ---- P1: G1 + G2 (all waves)
    // G1: delta[s][i] = (S_ref phi_s)[i] - v_s[i];  G2 (full walk): Kmat[tau][s] = psi_tau . phi_s,
    // weighted into Q[tau][s] = Ws[s, tau-1] Kmat[tau][s] by the producing lane.
    constexpr int NGW = kSegWaves;
    constexpr int NT1 = NTS * NTD, PER1 = (NT1 + NGW - 1) / NGW;
    constexpr int NT2 = FULL ? (CH / 16) * NTS : 0, PER2 = (NT2 + NGW - 1) / NGW;
    static_assert(!FULL || NT2 > 0, "G2 tiles");
    {
      // tile indices past the end are clamped (MFMAs stay unconditional, only the stores are guarded)
#pragma unroll 1
      for (int j = 0; j < PER1; ++j) {
        const int tile = min(wave + NGW * j, NT1 - 1);
        const bool valid = NT1 % NGW == 0 || wave + NGW * j < NT1;
        const int m0 = (tile % NTD) * 16, n0 = (tile / NTD) * 16;   // m: rows i, n: sources
        f32x4 acc = zero4();
#pragma unroll
        for (int k0 = 0; k0 < D; k0 += M::KS)
          acc = M::mma(frag_ld_row<T>(&sm.sref[0][0], D + 8, m0, k0), frag_ld_row<T>(&sm.phi[0][0], D + 8, n0, k0), acc);
        if (valid) {
          // rows i0..i0+3 of source s are contiguous in vd: v read and delta written in place
          const int s = n0 + (lane & 15), i0 = m0 + 4 * (lane >> 4);
          const int p = t0 - H + s;
          const bool src_ok = s < H + L && p >= 0;
          float d[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) d[r] = src_ok ? acc[r] - to_f32(sm.vd[s][i0 + r]) : 0.f;
          store4<T>(&sm.vd[s][i0], d[0], d[1], d[2], d[3]);
        }
      }
      if constexpr (FULL) {
        // G2 as transposed tiles (a lane holds sources s0..s0+3 of one target tau), weighted by
        // Ws[s, tau-1] into Q right away
#pragma unroll
        for (int j = 0; j < PER2; ++j) {
          const int tt = min(wave + NGW * j, NT2 - 1);
          const bool valid = NT2 % NGW == 0 || wave + NGW * j < NT2;
          const int m0 = (tt % NTS) * 16, n0 = (tt / NTS) * 16;   // m: sources s, n: targets tau
          f32x4 acc = zero4();
#pragma unroll
          for (int k0 = 0; k0 < D; k0 += M::KS)
            acc = M::mma(frag_ld_row<T>(&sm.phi[0][0], D + 8, m0, k0), frag_ld_row<T>(&sm.psi[0][0], D + 8, n0, k0), acc);
          if (valid) {
            const int t = n0 + (lane & 15), s0 = m0 + 4 * (lane >> 4);
            store4<T>(&sm.Q[t][s0], acc[0] * to_f32(sm.wsh[t][s0]), acc[1] * to_f32(sm.wsh[t][s0 + 1]),
                      acc[2] * to_f32(sm.wsh[t][s0 + 2]), acc[3] * to_f32(sm.wsh[t][s0 + 3]));
          }
        }
      }
    }
    __syncthreads();

    // ---- P3: G3 (y, full walk), then G4 + state update on the owned state tiles (all waves)
    if constexpr (FULL) {
      constexpr int NT3 = (CH / 16) * NTD, PER3 = (NT3 + kSegWaves - 1) / kSegWaves;
#pragma unroll 1
      for (int j = 0; j < PER3; ++j) {
        // past the end of the tile list the tile index is clamped (unconditional MFMAs, guarded stores)
        const int tile = min(wave + kSegWaves * j, NT3 - 1);
        const bool valid = NT3 % kSegWaves == 0 || wave + kSegWaves * j < NT3;
        {
          const int m0 = (tile % NTD) * 16, n0 = (tile / NTD) * 16;   // m: rows i, n: targets tau
          f32x4 aq = zero4(), as = zero4(), az = zero4();
#pragma unroll
          for (int k0 = 0; k0 < SPM; k0 += M::KS)
            aq = M::mma(frag_ld_tr<T>(&sm.vd[0][0], D + 8, m0, k0), frag_ld_row<T>(&sm.Q[0][0], SPM + 8, n0, k0), aq);
#pragma unroll
          for (int k0 = 0; k0 < D; k0 += M::KS) {
            const typename M::frag fb = frag_ld_row<T>(&sm.psi[0][0], D + 8, n0, k0);
            as = M::mma(frag_ld_row<T>(&sm.Sb[0][0], D + 8, m0, k0), fb, as);
            az = M::mma(frag_ld_row<T>(&sm.Zb[0][0], D + 8, m0, k0), fb, az);
          }
          // a lane holds rows i0..i0+3 of y for one target t
          const int t = n0 + (lane & 15), i0 = m0 + 4 * (lane >> 4);
          const float ac = sm.sc.acoef[t], kc = sm.sc.kcoef[t];
          float yv[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) yv[r] = -aq[r] + ac * as[r] - kc * az[r];
          if (bufchunk) {
            for (int s = 0; s < H; ++s) {
              const float* Bs = a.buf_in + ((size_t)bh * H + s) * D * D;
              f32x4 ab = zero4();
#pragma unroll
              for (int k0 = 0; k0 < D; k0 += M::KS)
                ab = M::mma(frag_ld<T>(Bs, D, 1, m0, k0), frag_ld_row<T>(&sm.psi[0][0], D + 8, n0, k0), ab);
              const float w = to_f32(sm.wsh[t][s]);
#pragma unroll
              for (int r = 0; r < 4; ++r) yv[r] -= w * ab[r];
            }
          }
          if (valid && t < L) store4<T>(a.y + (tb + t0 + t) * D + i0, yv[0], yv[1], yv[2], yv[3]);
        }
      }
    }
    if (owns) {
      // G4: U = -delta diag(Ws_end) phi^T, V = delta diag(Wz_end) phi^T, the end weights applied to the
      // delta fragments in registers; the full walk also forms the state after token Lmid - 1.
      const float a_end = sm.sc.endc[0], k_end = sm.sc.endc[1], b_end = sm.sc.endc[2];
      const bool do_clamp = !AGG && clamp_after(g, t1);
      const bool mid = FULL && g.Lmid > 0 && L > g.Lmid;
      const int m0 = mt * 16;
      constexpr int NKS = SPM / M::KS;
      if constexpr (FULL) {
        if (mid) {   // state after token Lmid - 1 (never a clamp point), from the chunk-start state
          float* rw_mid = rw + ((size_t)bh * g.ncb + (size_t)c * rb + 1) * 2 * D * D;
          typename M::frag fsm[NKS], fzm[NKS];
#pragma unroll
          for (int kk = 0; kk < NKS; ++kk) {
            const typename M::frag fd = frag_ld_tr<T>(&sm.vd[0][0], D + 8, m0, kk * M::KS);
            const int sb = kk * M::KS + (lane >> 4) * M::KL;
            fsm[kk] = frag_scale<T>(fd, &sm.sc.wsmid[sb]);
            fzm[kk] = frag_scale<T>(fd, &sm.sc.wzmid[sb]);
          }
#pragma unroll
          for (int jn = 0; jn < NOWN; ++jn) {
            const int n0 = (nt0 + jn) * 16;
            f32x4 aum = zero4(), avm = zero4();
#pragma unroll
            for (int kk = 0; kk < NKS; ++kk) {
              const typename M::frag fb = frag_ld_tr<T>(&sm.phi[0][0], D + 8, n0, kk * M::KS);
              aum = M::mma(fsm[kk], fb, aum);
              avm = M::mma(fzm[kk], fb, avm);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int i = m0 + 4 * (lane >> 4) + r, k = n0 + (lane & 15);
              float Um = -aum[r], Vm = avm[r];
              if (bufchunk) {
                for (int s = 0; s < H; ++s) {
                  const float b = a.buf_in[(((size_t)bh * H + s) * D + i) * D + k];
                  Um -= sm.sc.wsmid[s] * b;
                  Vm += sm.sc.wzmid[s] * b;
                }
              }
              rw_mid[(size_t)i * D + k] = sm.sc.midc[0] * Sr[jn][r] - sm.sc.midc[1] * Zr[jn][r] + Um;
              rw_mid[(size_t)D * D + (size_t)i * D + k] = g.momentum ? (sm.sc.midc[2] * Zr[jn][r] + Vm) : 0.f;
            }
          }
        }
      }
      typename M::frag fs[NKS], fz[NKS];
#pragma unroll
      for (int kk = 0; kk < NKS; ++kk) {
        const typename M::frag fd = frag_ld_tr<T>(&sm.vd[0][0], D + 8, m0, kk * M::KS);
        const int sb = kk * M::KS + (lane >> 4) * M::KL;
        fs[kk] = frag_scale<T>(fd, &sm.sc.wsend[sb]);
        fz[kk] = frag_scale<T>(fd, &sm.sc.wzend[sb]);
      }
      // raw end state -> the next chunk's saved start state (within the segment: the next segment's
      // workgroup writes its own start state, from the segment scan)
      float* rw_next = (FULL && c + 1 < c_end) ? rw + ((size_t)bh * g.ncb + (size_t)(c + 1) * rb) * 2 * D * D : nullptr;
#pragma unroll
      for (int jn = 0; jn < NOWN; ++jn) {
        const int n0 = (nt0 + jn) * 16;
        f32x4 au = zero4(), av = zero4();
#pragma unroll
        for (int kk = 0; kk < NKS; ++kk) {
          const typename M::frag fb = frag_ld_tr<T>(&sm.phi[0][0], D + 8, n0, kk * M::KS);
          au = M::mma(fs[kk], fb, au);
          av = M::mma(fz[kk], fb, av);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = m0 + 4 * (lane >> 4) + r, k = n0 + (lane & 15);
          float U = -au[r], V = av[r];
          if (bufchunk) {
            for (int s = 0; s < H; ++s) {
              const float b = a.buf_in[(((size_t)bh * H + s) * D + i) * D + k];
              U -= sm.sc.wsend[s] * b;
              V += sm.sc.wzend[s] * b;
            }
          }
          const float Sn = a_end * Sr[jn][r] - k_end * Zr[jn][r] + U;
          const float Zn = g.momentum ? (b_end * Zr[jn][r] + V) : 0.f;
          if (FULL && rw_next) {
            rw_next[(size_t)i * D + k] = Sn;
            rw_next[(size_t)D * D + (size_t)i * D + k] = Zn;
          }
          Sr[jn][r] = do_clamp ? clamp100(Sn) : Sn;
          Zr[jn][r] = Zn;
        }
      }
      if (FULL && clamp_point(g, t1)) {
        bool over = false;
#pragma unroll
        for (int jn = 0; jn < NOWN; ++jn)
#pragma unroll
          for (int r = 0; r < 4; ++r) over |= fabsf(Sr[jn][r]) > 100.f;
        flag_if_clamped(g, over);
      }
      if constexpr (AGG) {
        const float na = a_end * seg_a;
        const float nk = a_end * seg_k + k_end * seg_b;
        seg_b = b_end * seg_b;
        seg_a = na;
        seg_k = nk;
      }
    }
    if constexpr (FULL) {
      __syncthreads();                    // G3 done reading Sb / Zb
      if (owns) {
#pragma unroll
        for (int jn = 0; jn < NOWN; ++jn)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = mt * 16 + 4 * (lane >> 4) + r, k = (nt0 + jn) * 16 + (lane & 15);
            sm.Sb[i][k] = from_f32<T>(Sr[jn][r]);
            sm.Zb[i][k] = from_f32<T>(Zr[jn][r]);
          }
      }
    }
  }

  // ---- segment results
  if (owns) {
    if constexpr (AGG) {
      float* ag = agg + ((size_t)bh * sg.nseg + seg) * sg.agg_stride;
#pragma unroll
      for (int jn = 0; jn < NOWN; ++jn)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = mt * 16 + 4 * (lane >> 4) + r, k = (nt0 + jn) * 16 + (lane & 15);
          ag[(size_t)i * D + k] = Sr[jn][r];
          ag[(size_t)D * D + (size_t)i * D + k] = Zr[jn][r];
        }
      if (otile0 == 0 && lane == 0) {
        ag[2 * D * D] = seg_a; ag[2 * D * D + 1] = seg_k; ag[2 * D * D + 2] = seg_b;
      }
    } else if (FULL && seg == sg.nseg - 1) {
      // Sr holds the raw S_{T-1} (the last chunk of the sequence is never a clamp point)
#pragma unroll
      for (int jn = 0; jn < NOWN; ++jn)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = mt * 16 + 4 * (lane >> 4) + r, k = (nt0 + jn) * 16 + (lane & 15);
          const size_t off = sb + (size_t)i * D + k;
          a.S_T[off] = g.clamp_final ? clamp100(Sr[jn][r]) : Sr[jn][r];
          if (g.momentum) a.Z_T[off] = Zr[jn][r];
          if (final_raw) final_raw[off] = Sr[jn][r];
        }
    }
  }
}

}  // namespace atlas
