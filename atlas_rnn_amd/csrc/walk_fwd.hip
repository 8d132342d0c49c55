// walk_fwd.hip - specialised forward segment walks for bf16 inputs with d_k = d_v = 64.
//
// Same decomposition and outputs as seg_fwd.hip (segment aggregates -> segment scan -> full walk;
// chunk coefficients from k_chunk_coef), organised for a short per-chunk critical path:
//  * one workgroup barrier per chunk: the chunk inputs and the bf16 copy of the state are double
//    buffered in LDS, the next chunk's inputs are staged while the current one is computed, and the
//    chunk after that is already in flight in registers;
//  * wave w owns the state rows i in [16 (w & 3), +16) and, for the state update, the columns
//    k in [32 (w >> 2), +32), and computes y for the target tiles tau in [16 h, +16) and
//    [16 (3 - h), +16), h = w >> 2 (an early and a late tile: the products over sources are
//    formed on the causally nonzero source tiles only, so both halves do the same work);
//  * delta = S_ref phi - v and the weighted target/source products stay in registers between their
//    MFMAs (walk_common.h: chained operands), so only the staged inputs and the state copy go
//    through LDS;
//  * rows are read through per-row buffer resources: the halo before the first token and the
//    rows past T read as zeros, and y rows past T are dropped by the range check;
//  * a carried buffer (BUF): its sources are chunk 0's halo; their state terms (bufwalk.hip) are
//    added to the states after chunk 0 (its y terms are added after the walk).
// Sources of a chunk are the e - 1 halo tokens followed by the chunk's 64 tokens, s = 0 .. 79
// (window e <= 17); source s is token t0 - (e - 1) + s.
//
//   k_walk_agg  : zero initial state -> segment aggregate (a, kappa, b, U, V)       [WALK_AGG]
//   k_walk_full : from the segment-start state: y, S_T / Z_T, and the state at every backward-chunk
//                 boundary (chunk start and token Lmid - 1) for the backward, in the bf16 fragment
//                 layout of walk_common.h                                          [WALK_FULL]
#include "mem_common.h"
#include "mem_params.h"
#include "seg_common.h"
#include "walk_common.h"

namespace atlas {

namespace wf {

constexpr int D = 64;          // head size (d_k = d_v)
constexpr int CH = 64;         // chunk length
constexpr int SP = 80;         // source rows: halo (<= 16) + chunk
constexpr int NST = SP / 16;   // source tiles
constexpr int PD = D + 16;     // LDS pitch of D-wide rows (bf16)
constexpr int SPM = CH + kHaloPad;   // pitch of the coefficient arrays and Ws blocks in HBM (96)
constexpr int WP = SP + 8;     // LDS pitch of the Ws rows (88)
constexpr int REC = CoefRec<CH>::SIZE;   // 520 floats
// coefficient record offsets (floats)
constexpr int R_ACOEF = 0, R_KCOEF = CH, R_ENDC = 2 * CH, R_WSEND = 2 * CH + 4, R_WZEND = R_WSEND + SPM,
              R_WSMID = R_WZEND + SPM, R_WZMID = R_WSMID + SPM, R_MIDC = R_WZMID + SPM;
static_assert(R_MIDC + 4 == REC, "record layout");
static_assert((R_WSEND % 4) == 0 && (R_WZEND % 4) == 0 && (R_WSMID % 4) == 0 && (R_WZMID % 4) == 0, "float4 reads");
constexpr int NTH = kSegThreads;
constexpr int NV_SRC = SP * D / 8;     // 16-byte vectors of phi (or v) per chunk: 640
constexpr int NV_WSH = CH * SP / 8;    // 16-byte vectors of the Ws block rows we use: 640
constexpr int REC4 = REC / 4;          // 130

template <bool FULL>
struct Stage {
  alignas(16) bf16 phi[SP][PD];
  alignas(16) bf16 vv[SP][PD];
  alignas(16) bf16 psi[FULL ? CH : 1][PD];
  alignas(16) bf16 wsh[FULL ? CH : 1][WP];
  alignas(16) float rec[REC];
};

template <bool FULL>
struct Smem {
  Stage<FULL> st[2];
  alignas(16) bf16 SbT[FULL ? 2 : 1][FULL ? D : 1][PD];   // bf16 copy of S, transposed: SbT[k][i] = S[i][k]
  alignas(16) bf16 ZbT[FULL ? 2 : 1][FULL ? D : 1][PD];
};

// Per-thread register prefetch of one chunk (loads are unconditional; see walk_common.h).
template <bool FULL>
struct Prefetch {
  u32x4v phi[2], vv[2], psi, wsh[2], rec;
};

struct RowRes {
  rsrc_t k, v, q, rec, wsh;
};

// Per-thread constant offsets of the staged vectors.
struct StageOffs {
  uint32_t src[2];     // phi / v vector j: byte offset relative to token t0 (kOob for rows past the sources)
  uint32_t psi;
  uint32_t wsh[2];
  uint32_t rec;
  int lsrc[2];         // LDS element offsets (row * PD + col) or -1
  int lpsi;
  int lwsh[2];
};

__device__ __forceinline__ StageOffs stage_offsets(int H, int tid) {
  StageOffs o;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int v = tid + j * NTH;
    const int s = v >> 3, c8 = v & 7;
    const bool ok = v < NV_SRC && s < H + CH;
    o.src[j] = ok ? (uint32_t)((s - H) * (D * 2) + c8 * 16) : kOob;
    o.lsrc[j] = v < NV_SRC ? s * PD + c8 * 8 : -1;
  }
  o.psi = (uint32_t)((tid >> 3) * (D * 2) + (tid & 7) * 16);
  o.lpsi = (tid >> 3) * PD + (tid & 7) * 8;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int v = tid + j * NTH;
    const int t = v / (SP / 8), sv = v % (SP / 8);
    // Ws[s, t - 1] is zero for s > t + H - 1, that is past source tile (t >> 4) + 1 (H <= 16):
    // those vectors read as zeros (nothing is stored there)
    const bool nz = sv < 2 * ((t >> 4) + 2);
    o.wsh[j] = v < NV_WSH && nz ? (uint32_t)(t * SPM * 2 + sv * 16) : kOob;
    o.lwsh[j] = v < NV_WSH ? t * WP + sv * 8 : -1;
  }
  o.rec = tid < REC4 ? (uint32_t)(tid * 16) : kOob;
  return o;
}

template <bool FULL>
__device__ __forceinline__ void pf_load(Prefetch<FULL>& pf, const RowRes& rr, const StageOffs& o, int t0, int c) {
  const uint32_t tb = (uint32_t)t0 * (D * 2);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    pf.phi[j] = bld16(rr.k, o.src[j] + tb);
    pf.vv[j] = bld16(rr.v, o.src[j] + tb);
  }
  pf.rec = bld16(rr.rec, o.rec + (uint32_t)c * (REC * 4));
  if constexpr (FULL) {
    pf.psi = bld16(rr.q, o.psi + tb);
    const uint32_t wb = (uint32_t)c * (CH * SPM * 2);
#pragma unroll
    for (int j = 0; j < 2; ++j) pf.wsh[j] = bld16(rr.wsh, o.wsh[j] + wb);
  }
}

template <bool FULL, bool MAPE>
__device__ __forceinline__ void pf_store(const Prefetch<FULL>& pf, Stage<FULL>& st, const StageOffs& o, int tid,
                                         int deg) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    if (o.lsrc[j] >= 0) {
      u32x4v x = pf.phi[j];
      if constexpr (MAPE) x = map_bf16x8(x, deg);
      *reinterpret_cast<u32x4v*>(&st.phi[0][0] + o.lsrc[j]) = x;
      *reinterpret_cast<u32x4v*>(&st.vv[0][0] + o.lsrc[j]) = pf.vv[j];
    }
  }
  if (tid < REC4) *reinterpret_cast<u32x4v*>(&st.rec[tid * 4]) = pf.rec;
  if constexpr (FULL) {
    u32x4v x = pf.psi;
    if constexpr (MAPE) x = map_bf16x8(x, deg);
    *reinterpret_cast<u32x4v*>(&st.psi[0][0] + o.lpsi) = x;
#pragma unroll
    for (int j = 0; j < 2; ++j)
      if (o.lwsh[j] >= 0) *reinterpret_cast<u32x4v*>(&st.wsh[0][0] + o.lwsh[j]) = pf.wsh[j];
  }
}

// Accumulator tile idx of a, or zeros past the last tile (idx is a compile-time constant after unrolling).
template <int N>
__device__ __forceinline__ f32x4 tile_or_zero(const f32x4 (&a)[N], int idx) {
  return idx < N ? a[idx < N ? idx : 0] : zero4();
}

}  // namespace wf

// One segment of one row. FULL = false: aggregate pass; FULL = true: full walk.
// TH = 0, 1 (full walks): the wave's column half as a constant, target tiles TH and 3 - TH, and
// products over the source tiles that reach them only (y_tau takes sources s <= tau + H - 1, that
// is tiles S <= T + 1 of target tile T); TH = 2: the half at run time, target tiles 2 h, 2 h + 1
// and every source tile (the carried-buffer walks, whose registers have no room for the pruned
// bodies).
template <bool FULL, bool MAPE, bool BUF, int TH = 2>
__device__ __forceinline__ void walk_fwd(const Geom& g, const FwdPtrs<bf16>& a, const SegGeom& sg, float* agg,
                                         const float* seg_states, float* rw, float* final_raw, const float* coef,
                                         const bf16* wsh_all, unsigned char* smem_raw) {
  using namespace wf;
  typedef Smem<FULL> Sm;
  Sm& sm = *reinterpret_cast<Sm*>(smem_raw);
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int gq = lane >> 4, m = lane & 15;
  const int it = wave & 3, th = TH < 2 ? TH : wave >> 2;   // state rows 16 it ..; column half th
  const int TT[2] = {TH < 2 ? TH : 2 * th, TH < 2 ? 3 - TH : 2 * th + 1};   // target tiles
  constexpr int NK[2] = {TH == 0 ? 2 : TH == 1 ? 3 : NST, TH == 0 ? NST : TH == 1 ? 4 : NST};
  const int seg = blockIdx.x, bh = blockIdx.y;
  const int H = g.H;
  const int c_begin = seg * sg.G, c_end = min(g.nc, c_begin + sg.G);
  const size_t DD = (size_t)D * D;

  RowRes rr;
  const uint32_t row_bytes = (uint32_t)g.T * (D * 2);
  rr.k = make_rsrc(a.k + (size_t)bh * g.T * D, row_bytes);
  rr.v = make_rsrc(a.v + (size_t)bh * g.T * D, row_bytes);
  rr.q = make_rsrc(a.q + (size_t)bh * g.T * D, row_bytes);
  rr.rec = make_rsrc(coef + (size_t)bh * g.nc * REC, (uint32_t)g.nc * (REC * 4));
  rr.wsh = make_rsrc(FULL ? wsh_all + (size_t)bh * g.nc * CH * SPM : nullptr,
                     FULL ? (uint32_t)g.nc * (CH * SPM * 2) : 0u);
  const StageOffs so = stage_offsets(H, tid);
  const rsrc_t ry = make_rsrc(FULL ? a.y + (size_t)bh * g.T * D : nullptr, FULL ? row_bytes : 0u);

  // the first chunk's loads go out before those of S_ref and the segment-start state, so that the
  // walk's start waits for one round trip to memory instead of two
  Prefetch<FULL> pf;
  if (c_begin < c_end) pf_load<FULL>(pf, rr, so, c_begin * CH, c_begin);

  // S_ref rows 16 it .. +15 as the B operand of delta^T = phi S_ref^T (k = 32 q + 8 gq + e)
  bf16x8 sref_f[2];
  {
    const float* sr = a.S_ref + (size_t)bh * DD + (size_t)(16 * it + m) * D;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const float4 x0 = *reinterpret_cast<const float4*>(sr + 32 * q + 8 * gq);
      const float4 x1 = *reinterpret_cast<const float4*>(sr + 32 * q + 8 * gq + 4);
      bf16x8 f;
      f[0] = static_cast<bf16>(x0.x); f[1] = static_cast<bf16>(x0.y); f[2] = static_cast<bf16>(x0.z);
      f[3] = static_cast<bf16>(x0.w); f[4] = static_cast<bf16>(x1.x); f[5] = static_cast<bf16>(x1.y);
      f[6] = static_cast<bf16>(x1.z); f[7] = static_cast<bf16>(x1.w);
      sref_f[q] = f;
    }
  }

  // owned state tiles: rows i = 16 it + 4 gq + r, columns k = 32 th + 16 j + m
  float Sr[2][4], Zr[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) { Sr[j][r] = 0.f; Zr[j][r] = 0.f; }
  float seg_a = 1.f, seg_k = 0.f, seg_b = 1.f;
  const int i0 = 16 * it + 4 * gq;
  const int rb = g.Lmid > 0 ? 2 : 1;
  // saved states (walk_common.h layout): block of backward chunk cb at rw_row + cb * kStateBlk
  // (rows of g.ncb blocks with mid points; of g.nc blocks, one per chunk, without)
  unsigned char* rw_row =
      FULL ? reinterpret_cast<unsigned char*>(rw) + (size_t)bh * (rb == 2 ? g.ncb : g.nc) * kStateBlk : nullptr;
  // this lane's 8-byte half of the fragments of its tiles j = 0, 1
  const uint32_t f2o[2] = {frag_off(2 * th, it >> 1, lane) + (it & 1) * 8,
                           frag_off(2 * th + 1, it >> 1, lane) + (it & 1) * 8};
  auto save_state = [&](int cb, const float (&Sv)[2][4], const float (&Zv)[2][4]) {
    unsigned char* blk = rw_row + (size_t)cb * kStateBlk;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      *reinterpret_cast<uint2*>(blk + f2o[j]) =
          make_uint2(pack_bf16x2(Sv[j][0], Sv[j][1]), pack_bf16x2(Sv[j][2], Sv[j][3]));
      *reinterpret_cast<uint2*>(blk + kStateBytes + f2o[j]) =
          make_uint2(pack_bf16x2(Zv[j][0], Zv[j][1]), pack_bf16x2(Zv[j][2], Zv[j][3]));
    }
  };

  if constexpr (FULL) {
    const float* ss = seg_states + ((size_t)bh * sg.nseg + seg) * 2 * DD;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int k = 32 * th + 16 * j + m;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const size_t off = (size_t)(i0 + r) * D + k;
        Sr[j][r] = ss[off];
        Zr[j][r] = ss[DD + off];
      }
      store4<bf16>(&sm.SbT[0][k][i0], Sr[j][0], Sr[j][1], Sr[j][2], Sr[j][3]);
      store4<bf16>(&sm.ZbT[0][k][i0], Zr[j][0], Zr[j][1], Zr[j][2], Zr[j][3]);
    }
    save_state(c_begin * rb, Sr, Zr);
  }

  if (c_begin < c_end) {
    pf_store<FULL, MAPE>(pf, sm.st[0], so, tid, g.map_deg);
    if (c_begin + 1 < c_end) pf_load<FULL>(pf, rr, so, (c_begin + 1) * CH, c_begin + 1);
  }
  __syncthreads();

  for (int c = c_begin; c < c_end; ++c) {
    const int b = (c - c_begin) & 1;
    const Stage<FULL>& st = sm.st[b];
    const int t0 = c * CH;
    const int L = min(g.T, t0 + CH) - t0;

    // ---- delta^T[s][i] for all sources, rows i of this wave; (FULL) K^T[s][tau] = phi_s . psi_tau
    f32x4 dl[NST];
    f32x4 kq[FULL ? 2 : 1][NST];
    bf16x8 psf[FULL ? 2 : 1][2];
    if constexpr (FULL) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int q = 0; q < 2; ++q) psf[u][q] = frag_row(&st.psi[0][0], PD, 16 * TT[u], 32 * q);
    }
#pragma unroll
    for (int s4 = 0; s4 < NST; ++s4) {
      dl[s4] = zero4();
      if constexpr (FULL) { kq[0][s4] = zero4(); kq[1][s4] = zero4(); }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const bf16x8 fa = frag_row(&st.phi[0][0], PD, 16 * s4, 32 * q);
        dl[s4] = mma_bf16(fa, sref_f[q], dl[s4]);
        if constexpr (FULL) {
          if (s4 < NK[0]) kq[0][s4] = mma_bf16(fa, psf[0][q], kq[0][s4]);
          if (s4 < NK[1]) kq[1][s4] = mma_bf16(fa, psf[1][q], kq[1][s4]);
        }
      }
    }
    // delta = acc - v  (lane: sources 16 s4 + 4 gq + r, row i = 16 it + m)
#pragma unroll
    for (int s4 = 0; s4 < NST; ++s4) {
      const s16x4 vt = tr4(&st.vv[0][0], PD, 16 * s4, 16 * it);
#pragma unroll
      for (int r = 0; r < 4; ++r) dl[s4][r] -= bf16_bits_to_f32((unsigned short)vt[r]);
    }

    const float* rec = st.rec;
    // the carried buffer's first-chunk terms (bufwalk.hip), chunk 0 of a call with a buffer only
    const float* bufc = (BUF && c == 0) ? a.buf_corr + (size_t)bh * bufw::kCorrFloats : nullptr;
    // chained operands over the source slots of k-step q: tiles 2q (slots 0..3) and 2q+1 (4..7)
    constexpr int NQ = (NST + 1) / 2;   // 3
    bf16x8 fws[NQ], fwz[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const f32x4 lo = tile_or_zero(dl, 2 * q + 1);
      const float4 whi = *reinterpret_cast<const float4*>(rec + R_WSEND + 32 * q + 4 * gq);
      const float4 wlo = *reinterpret_cast<const float4*>(rec + R_WSEND + 32 * q + 16 + 4 * gq);
      const float4 zhi = *reinterpret_cast<const float4*>(rec + R_WZEND + 32 * q + 4 * gq);
      const float4 zlo = *reinterpret_cast<const float4*>(rec + R_WZEND + 32 * q + 16 + 4 * gq);
      fws[q] = pack_frag_scaled(dl[2 * q], lo, whi, wlo);
      fwz[q] = pack_frag_scaled(dl[2 * q], lo, zhi, zlo);
    }

    // ---- y (FULL): y^T tile C[i][tau] = sum_s delta[i][s] Q[tau][s] + a psi S^T - kappa psi Z^T
    if constexpr (FULL) {
      const int sbuf = b;
      bf16x8 fdl[NQ];
#pragma unroll
      for (int q = 0; q < NQ; ++q) fdl[q] = pack_frag(dl[2 * q], tile_or_zero(dl, 2 * q + 1));
      bf16x8 fS[2], fZ[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        fS[q] = frag_ld_tr<bf16>(&sm.SbT[sbuf][0][0], PD, 16 * it, 32 * q);
        fZ[q] = frag_ld_tr<bf16>(&sm.ZbT[sbuf][0][0], PD, 16 * it, 32 * q);
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int tt = TT[u];
        // Q[tau][s] = Ws[s, tau-1] K[tau][s]; lane: tau = 16 tt + m, sources 16 s4 + 4 gq + r
        f32x4 qv[NST];
#pragma unroll
        for (int s4 = 0; s4 < NST; ++s4) {
          if (s4 < NK[u]) {
            const float4 w = lds_bf16x4(&st.wsh[16 * tt + m][16 * s4 + 4 * gq]);
            qv[s4][0] = kq[u][s4][0] * w.x; qv[s4][1] = kq[u][s4][1] * w.y;
            qv[s4][2] = kq[u][s4][2] * w.z; qv[s4][3] = kq[u][s4][3] * w.w;
          } else {
            qv[s4] = zero4();
          }
        }
        f32x4 aq = zero4(), as = zero4(), az = zero4();
#pragma unroll
        for (int q = 0; q < NQ; ++q)
          if (2 * q < NK[u]) aq = mma_bf16(fdl[q], pack_frag(qv[2 * q], tile_or_zero(qv, 2 * q + 1)), aq);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          as = mma_bf16(fS[q], psf[u][q], as);
          az = mma_bf16(fZ[q], psf[u][q], az);
        }
        const int tau = 16 * tt + m;
        const float ac = rec[R_ACOEF + tau], kc = rec[R_KCOEF + tau];
        u32x2v out;
        out[0] = pack_bf16x2(-aq[0] + ac * as[0] - kc * az[0], -aq[1] + ac * as[1] - kc * az[1]);
        out[1] = pack_bf16x2(-aq[2] + ac * as[2] - kc * az[2], -aq[3] + ac * as[3] - kc * az[3]);
        bst8(ry, (uint32_t)(((t0 + tau) * D + i0) * 2), out);
      }
    }

    // ---- state update on the owned tiles: U = -delta diag(Ws_end) phi, V = delta diag(Wz_end) phi
    {
      const float a_end = rec[R_ENDC], k_end = rec[R_ENDC + 1], b_end = rec[R_ENDC + 2];
      bf16x8 fb[2][NQ];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int kcol = 32 * th + 16 * j;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          if (32 * q + 16 < SP) fb[j][q] = tr_pair<true>(&st.phi[0][0], PD, q, kcol);
          else fb[j][q] = tr_pair<false>(&st.phi[0][0], PD, q, kcol);
        }
      }
      const bool mid = FULL && g.Lmid > 0 && L > g.Lmid;
      if constexpr (FULL) {
        if (mid) {   // state after token Lmid - 1 (a backward-chunk boundary)
          bf16x8 fsm[NQ], fzm[NQ];
#pragma unroll
          for (int q = 0; q < NQ; ++q) {
            const f32x4 lo = tile_or_zero(dl, 2 * q + 1);
            const float4 whi = *reinterpret_cast<const float4*>(rec + R_WSMID + 32 * q + 4 * gq);
            const float4 wlo = *reinterpret_cast<const float4*>(rec + R_WSMID + 32 * q + 16 + 4 * gq);
            const float4 zhi = *reinterpret_cast<const float4*>(rec + R_WZMID + 32 * q + 4 * gq);
            const float4 zlo = *reinterpret_cast<const float4*>(rec + R_WZMID + 32 * q + 16 + 4 * gq);
            fsm[q] = pack_frag_scaled(dl[2 * q], lo, whi, wlo);
            fzm[q] = pack_frag_scaled(dl[2 * q], lo, zhi, zlo);
          }
          const float ma = rec[R_MIDC], mk = rec[R_MIDC + 1], mb = rec[R_MIDC + 2];
          float Sm_[2][4], Zm_[2][4];
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            f32x4 au = zero4(), av = zero4();
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
              au = mma_bf16(fsm[q], fb[j][q], au);
              av = mma_bf16(fzm[q], fb[j][q], av);
            }
            const int kk = 32 * th + 16 * j + m;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              Sm_[j][r] = ma * Sr[j][r] - mk * Zr[j][r] - au[r];
              Zm_[j][r] = g.momentum ? (mb * Zr[j][r] + av[r]) : 0.f;
              if (BUF && bufc) {
                Sm_[j][r] += bufc[bufw::SM + (i0 + r) * D + kk];
                Zm_[j][r] += bufc[bufw::ZM + (i0 + r) * D + kk];
              }
            }
          }
          save_state(c * rb + 1, Sm_, Zm_);
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        f32x4 au = zero4(), av = zero4();
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          au = mma_bf16(fws[q], fb[j][q], au);
          av = mma_bf16(fwz[q], fb[j][q], av);
        }
        const int k = 32 * th + 16 * j + m;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float Sn = a_end * Sr[j][r] - k_end * Zr[j][r] - au[r];
          const float Zn = g.momentum ? (b_end * Zr[j][r] + av[r]) : 0.f;
          Sr[j][r] = Sn;
          Zr[j][r] = Zn;
        }
        if constexpr (FULL) {
          store4<bf16>(&sm.SbT[b ^ 1][k][i0], Sr[j][0], Sr[j][1], Sr[j][2], Sr[j][3]);
          store4<bf16>(&sm.ZbT[b ^ 1][k][i0], Zr[j][0], Zr[j][1], Zr[j][2], Zr[j][3]);
        }
      }
      if constexpr (BUF) {
        if (bufc) {   // chunk 0: the buffer sources' terms of the end state (and its bf16 copy again)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int k = 32 * th + 16 * j + m;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              Sr[j][r] += bufc[bufw::SE + (i0 + r) * D + k];
              Zr[j][r] += bufc[bufw::ZE + (i0 + r) * D + k];
            }
            if constexpr (FULL) {
              store4<bf16>(&sm.SbT[b ^ 1][k][i0], Sr[j][0], Sr[j][1], Sr[j][2], Sr[j][3]);
              store4<bf16>(&sm.ZbT[b ^ 1][k][i0], Zr[j][0], Zr[j][1], Zr[j][2], Zr[j][3]);
            }
          }
        }
      }
      if constexpr (FULL) {
        if (clamp_point(g, t0 + L)) {
          bool over = false;
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) over |= fabsf(Sr[j][r]) > 100.f;
          flag_if_clamped(g, over);
        }
      }
      if constexpr (FULL) {
        if (c + 1 < c_end) save_state((c + 1) * rb, Sr, Zr);
      }
      if constexpr (!FULL) {
        const float na = a_end * seg_a;
        const float nk = a_end * seg_k + k_end * seg_b;
        seg_b = b_end * seg_b;
        seg_a = na;
        seg_k = nk;
      }
    }

    // ---- stage the next chunk, start loading the one after
    if (c + 1 < c_end) {
      pf_store<FULL, MAPE>(pf, sm.st[b ^ 1], so, tid, g.map_deg);
      if (c + 2 < c_end) pf_load<FULL>(pf, rr, so, (c + 2) * CH, c + 2);
    }
    __syncthreads();
  }

  // ---- segment results
  if constexpr (!FULL) {
    float* ag = agg + ((size_t)bh * sg.nseg + seg) * sg.agg_stride;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const size_t off = (size_t)(i0 + r) * D + 32 * th + 16 * j + m;
        ag[off] = Sr[j][r];
        ag[DD + off] = Zr[j][r];
      }
    if (tid == 0) { ag[2 * DD] = seg_a; ag[2 * DD + 1] = seg_k; ag[2 * DD + 2] = seg_b; }
  } else {
    if (seg == sg.nseg - 1) {
      const size_t sb = (size_t)bh * DD;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const size_t off = sb + (size_t)(i0 + r) * D + 32 * th + 16 * j + m;
          a.S_T[off] = g.clamp_final ? clamp100(Sr[j][r]) : Sr[j][r];
          if (g.momentum) a.Z_T[off] = Zr[j][r];
          if (final_raw) final_raw[off] = Sr[j][r];
        }
    }
  }
}

// (a carried buffer's terms reach segment 0's aggregate in the segment scan, not here)
template <bool MAPE>
__global__ __launch_bounds__(kSegThreads) __attribute__((amdgpu_waves_per_eu(4))) void k_walk_agg(
    const Geom g, const FwdPtrs<bf16> a, const SegGeom sg, float* agg, const float* coef) {
  if (geom_skip(g)) return;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  walk_fwd<false, MAPE, false>(g, a, sg, agg, nullptr, nullptr, nullptr, coef, nullptr, smem_raw);
}

template <bool MAPE, bool BUF>
__global__ __launch_bounds__(kSegThreads) void k_walk_full(const Geom g, const FwdPtrs<bf16> a, const SegGeom sg,
                                                             const float* seg_states, float* rw, float* final_raw,
                                                             const float* coef, const bf16* wsh) {
  if (geom_skip(g)) return;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  if constexpr (BUF)
    walk_fwd<true, MAPE, BUF>(g, a, sg, nullptr, seg_states, rw, final_raw, coef, wsh, smem_raw);
  else if (__builtin_amdgcn_readfirstlane(wave_id() >> 2) == 0)
    walk_fwd<true, MAPE, BUF, 0>(g, a, sg, nullptr, seg_states, rw, final_raw, coef, wsh, smem_raw);
  else
    walk_fwd<true, MAPE, BUF, 1>(g, a, sg, nullptr, seg_states, rw, final_raw, coef, wsh, smem_raw);
}

template <typename T, int D>
hipError_t launch_fwd_seg_scan(const Geom& g, const FwdPtrs<T>& a, const SegGeom& sg, const float* agg,
                               float* seg_states, hipStream_t stream);

// The specialised walks cover bf16, d = 64, window <= 17 and no clamp at scan_chunk_len boundaries
// (a carried buffer enters through bufwalk.hip's first-chunk terms); everything else runs through
// seg_fwd.hip.
bool walk_fwd_supported(const Geom& g) {
  return g.DK == 64 && g.DV == 64 && g.Lc == wf::CH && g.H <= wf::SP - wf::CH && g.clamp_every == 0;
}

template <bool MAPE, bool BUF>
static hipError_t launch_walks(const Geom& g, const FwdPtrs<bf16>& a, const SegGeom& sg, float* agg,
                               float* seg_states, float* rw, float* final_raw, float* coef, bf16* wsh,
                               hipStream_t stream) {
  hipError_t err;
  if (sg.nseg > 1) {
    const size_t smem = sizeof(wf::Smem<false>);
    err = set_dyn_smem(reinterpret_cast<const void*>(&k_walk_agg<MAPE>), smem);
    if (err != hipSuccess) return err;
    prof_name(KID_FWD_SEG_AGG, "k_walk_agg");
    prof_begin(KID_FWD_SEG_AGG, stream);
    hipLaunchKernelGGL((k_walk_agg<MAPE>), dim3(sg.nseg, g.BH), dim3(kSegThreads), smem, stream, g, a, sg, agg,
                       (const float*)coef);
    prof_end(KID_FWD_SEG_AGG, stream);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  if ((err = launch_fwd_seg_scan<bf16, 64>(g, a, sg, agg, seg_states, stream)) != hipSuccess) return err;
  const size_t smem = sizeof(wf::Smem<true>);
  err = set_dyn_smem(reinterpret_cast<const void*>(&k_walk_full<MAPE, BUF>), smem);
  if (err != hipSuccess) return err;
  prof_name(KID_FWD_WALK, "k_walk_full");
  prof_begin(KID_FWD_WALK, stream);
  hipLaunchKernelGGL((k_walk_full<MAPE, BUF>), dim3(sg.nseg, g.BH), dim3(kSegThreads), smem, stream, g, a, sg,
                     (const float*)seg_states, rw, final_raw, (const float*)coef, (const bf16*)wsh);
  prof_end(KID_FWD_WALK, stream);
  return hipGetLastError();
}

hipError_t launch_walk_fwd(const Geom& g, const FwdPtrs<bf16>& a, const SegGeom& sg, float* agg, float* seg_states,
                           float* rw, float* final_raw, float* coef, bf16* wsh, hipStream_t stream) {
  // the chunk coefficient records (coef, wsh) are formed by the caller first
  const bool mape = g.map_mode == MAP_ELEMENTWISE, buf = a.buf_corr != nullptr;
  if (buf)
    return mape ? launch_walks<true, true>(g, a, sg, agg, seg_states, rw, final_raw, coef, wsh, stream)
                : launch_walks<false, true>(g, a, sg, agg, seg_states, rw, final_raw, coef, wsh, stream);
  return mape ? launch_walks<true, false>(g, a, sg, agg, seg_states, rw, final_raw, coef, wsh, stream)
              : launch_walks<false, false>(g, a, sg, agg, seg_states, rw, final_raw, coef, wsh, stream);
}

}  // namespace atlas
