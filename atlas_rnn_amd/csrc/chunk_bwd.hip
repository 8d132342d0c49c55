// chunk_bwd.hip - reverse walk of the backward pass with every coefficient formed in the kernel
// (bf16 inputs, d_k = d_v = 64, window <= 17, no scan_chunk_len clamp, no carried buffer).
//
// One workgroup of 8 waves per (segment, row); the segments are the forward's (G chunks of 64
// tokens). The adjoint at each segment end comes from the adjoint aggregates and their scan
// (seg_bwd.hip); the boundary merge and the dS_ref sum are the shared fixup (seg_fixup.h).
//
//   forward pass over the segment: the chunk-start states X_c = (S_c, Z_c) from the segment-start
//     state (X_{c+1} = T_c X_c + (U_c, V_c)), kept in the workspace as bf16 (16 KB per chunk, read
//     back by the same workgroup) with each chunk's end coefficients (a record of 292 floats);
//   reverse pass, chunk c (targets t = 0 .. 63, sources s = 0 .. 79 at tokens t0 - 16 + s), with
//   Lam = (lamS, lamZ) the adjoint of (S, Z) after the chunk's last token:
//     dpsi_t  = S_{t-1}^T dy_t = At S_c^T dy_t + Kt Z_c^T dy_t + sum_s R[s][t] phi_s
//     ddelta_s = sum_t Q[s][t] dy_t + cs_s lamS phi_s + cz_s lamZ phi_s
//     dphi_s  = sum_t R[s][t] psi_t + cs_s lamS^T delta_s + cz_s lamZ^T delta_s + S_ref^T ddelta_s
//     with K[s][t] = phi_s . psi_t, Dd[s][t] = delta_s . dy_t, Wy[s][t] the coefficient of
//     G_s = delta_s phi_s^T in S_{t-1}, Q = K o Wy, R = Dd o Wy;
//   the scalar gradients are inner products of the adjoint at t with the state at t - 1. Both are
//     combinations of a few bases: adjoint bases E_q = dy_q psi_q^T (q > t), lamS, lamZ; state
//     bases G_s, S_c, Z_c. Their Gram matrix M (M[q][s] = K[s][q] Dd[s][q]; fS, fZ; hS, hZ; the
//     four state-adjoint Grams) is contracted on the matrix cores with the adjoint coefficients
//     (Am[t][q] = A(t -> q-1) for lamS_t; C'[t][q] for the total lamZ_t = d/dg_t) and then with
//     the state coefficients (Wy; Wzy: of G_s in Z_{t-1}):
//       dalpha_t = <lamS_t, S_{t-1}>,  deta_t = -<lamS_t, Z_t> = -(beta_t <lamS_t, Z_{t-1}> + <lamS_t, g_t>),
//       dbeta_t = <lamZ_t, Z_{t-1}>,   dw[t][j] = <lamZ_t, G_{t-j}>;
//   then Lam <- T_c^T Lam + sum_t (At, Kt) E_t.
// The halo sources of chunk c are the last 16 tokens of chunk c - 1: their partial gradients stay
// in the registers of the lanes that hold those tokens' rows in the next step.
#include "chunk_common.h"
#include "seg_fixup.h"

namespace atlas {

namespace cpb {
using namespace cp;

constexpr int NTB = 512;

// The thread index through an empty asm: values derived from it inside the walk's loops are
// recomputed where they are used instead of being hoisted out of the loop and held in registers
// for its whole length.
__device__ __forceinline__ int fresh_tid() { return launder((int)threadIdx.x); }
#define CPB_FRESH_LANE                                                  \
  const int tid = fresh_tid(), lane = tid & 63, gq = lane >> 4, m = lane & 15; \
  (void)tid; (void)lane; (void)gq; (void)m;
constexpr int NWB = NTB / 64;
constexpr int PB = 72;    // LDS pitch (bf16 elements) of 64-wide rows
constexpr int QP = 88;    // pitch of the Q^T / R^T rows [t][s] (80 sources + 8)
constexpr int MP = 104;   // pitch of the Gram rows [q][s'] (96 state bases + 8)
constexpr int EMAX = 17;  // window
// chunk coefficient record (floats): cs, cz (sources), cgS, cgZ (targets), the chunk transition
constexpr int R_CS = 0, R_CZ = SRC, R_GS = 2 * SRC, R_GZ = 2 * SRC + CL, R_TR = 2 * SRC + 2 * CL;
constexpr int REC = R_TR + 4;   // 292
static_assert(REC <= NTB, "one record element per thread");
// workspace per chunk between the passes: S_c^T, Z_c^T (bf16) and the coefficient record
constexpr size_t kXsStates = (size_t)2 * D * D * 2;
constexpr size_t kXsBytes = kXsStates + ((REC * 4 + 255) / 256) * 256;

struct BwSm;
struct BwSm {
  alignas(16) bf16 phi[SRC][PB];     // sources (mapped)
  alignas(16) bf16 psi[CL][PB];      // targets (mapped)
  alignas(16) bf16 dy[CL][PB];
  alignas(16) bf16 vd[SRC][PB];      // v; delta (reverse pass); ddelta (after the s-phase)
  alignas(16) bf16 XS[2][D][PB];     // S_c^T, Z_c^T   ([k][i])
  alignas(16) bf16 XL[2][D][PB];     // lamS^T, lamZ^T ([k][i])
  alignas(16) bf16 Qt[CL][QP];       // Q[s][t] stored [t][s]
  alignas(16) bf16 Rt[CL][QP];
  alignas(16) bf16 Mt[CL][MP];       // Gram M[q][s'] (q: adjoint basis E_q; s' < 80: G_s, 80: S_c, 81: Z_c)
  alignas(16) bf16 Cb[CL][PB];       // C'[r][t]: of g_r in S_{t-1} (r, t chunk-local targets)
  alignas(16) float co[REC];
  alignas(16) float la[CL], lb[CL], eta[CL], At[CL], Kt[CL], B1[CL], be[CL];
  float hp[2][4][SRC];               // hS / hZ partials by column tile
  float gram[NWB][4];
  // the window band Bd[s][r] = w(r, r + HT - s) (0 <= r + HT - s < e; zero elsewhere): the weight of
  // source s in the window of target r, i.e. of lag j = r + HT - s (w: the lag gate, the token gate
  // of the source, or 1; zero for targets past T)
  alignas(16) bf16 Bd[SRC][PB];
  // end terms of ddelta / dphi (waves 4-7), bf16 pairs in the accumulator layout: [ct][st][pair][lane]
  unsigned ed[4][SRC / 16][2][64], ef[4][SRC / 16][2][64];
};

static_assert(sizeof(BwSm) <= 160 * 1024, "one workgroup per CU: at most 160 KB of LDS");

// register prefetch of one chunk's rows in wave-loads of 8 rows (64 lanes x 16 bytes): wave-load j
// = w + 8 u of wave w. j < 10: phi rows t0 - 16 + 8 j ..; < 20: v rows; < 28: psi rows t0 + ..; < 36:
// dy rows. The kind of a wave-load is uniform over the wave (scalar branches; the rows before token
// 0 read as zeros: their offsets lie outside the buffer resource).
constexpr int WL_F = 2 * SRC / 8;            // 20: phi, v [forward pass]
constexpr int WL_R = WL_F + 2 * CL / 8;      // 36: + psi, dy [reverse pass]
template <int NWL>
struct RowPf { u32x4v v[(NWL + NWB - 1) / NWB]; };

template <int NWL>
__device__ __forceinline__ void rows_load(RowPf<NWL>& pf, rsrc_t rk, rsrc_t rv, rsrc_t rq, rsrc_t rdy, int t0, int w) {
  const int lane = fresh_tid() & 63;
  const uint32_t lo = (uint32_t)((lane >> 3) * (D * 2) + (lane & 7) * 16);
#pragma unroll
  for (int u = 0; u < (NWL + NWB - 1) / NWB; ++u) {
    const int j = w + NWB * u;
    if (j < NWL) {
      if (j < SRC / 8) pf.v[u] = bld16(rk, (uint32_t)((t0 - HT + 8 * j) * (D * 2)) + lo);
      else if (j < 2 * SRC / 8) pf.v[u] = bld16(rv, (uint32_t)((t0 - HT + 8 * (j - SRC / 8)) * (D * 2)) + lo);
      else if (j < 2 * SRC / 8 + CL / 8) pf.v[u] = bld16(rq, (uint32_t)((t0 + 8 * (j - 2 * SRC / 8)) * (D * 2)) + lo);
      else pf.v[u] = bld16(rdy, (uint32_t)((t0 + 8 * (j - 2 * SRC / 8 - CL / 8)) * (D * 2)) + lo);
    }
  }
}
template <bool MAPE, int NWL>
__device__ __forceinline__ void rows_store(const RowPf<NWL>& pf, BwSm& sm, int deg, int w) {
  const int lane = fresh_tid() & 63;
  const int rr = lane >> 3, cc = (lane & 7) * 8;
#pragma unroll
  for (int u = 0; u < (NWL + NWB - 1) / NWB; ++u) {
    const int j = w + NWB * u;
    if (j < NWL) {
      u32x4v x = pf.v[u];
      bf16* dst;
      if (j < SRC / 8) {
        if constexpr (MAPE) x = map_bf16x8(x, deg);
        dst = &sm.phi[8 * j + rr][cc];
      } else if (j < 2 * SRC / 8) {
        dst = &sm.vd[8 * (j - SRC / 8) + rr][cc];
      } else if (j < 2 * SRC / 8 + CL / 8) {
        if constexpr (MAPE) x = map_bf16x8(x, deg);
        dst = &sm.psi[8 * (j - 2 * SRC / 8) + rr][cc];
      } else {
        dst = &sm.dy[8 * (j - 2 * SRC / 8 - CL / 8) + rr][cc];
      }
      *reinterpret_cast<u32x4v*>(dst) = x;
    }
  }
}

// the (segment, row) block of a boundary-partial buffer [BH][nseg][H][2D]
__device__ __forceinline__ float* part_row(float* base, int bh, int nseg, int seg, int H) {
  return base + ((size_t)bh * nseg + seg) * H * (2 * D);
}

// the chunk's scalars (wave 0: lane = target) and gates (raw bf16 bits)
struct ScalPf {
  unsigned short al, et, be;
  unsigned short gt[3];
};
__device__ __forceinline__ void scal_load(ScalPf& p, const Geom& g, const BwdPtrs<bf16>& a, size_t rowbase, int t0) {
  const int tid = fresh_tid();
  p.al = 0x3f80; p.et = 0; p.be = 0x3f80;   // 1, 0, 1 (the identity past T)
  if (tid < 64 && t0 + tid < g.T) {
    const size_t o = rowbase + t0 + tid;
    p.al = __builtin_bit_cast(unsigned short, a.decay[o]);
    p.et = __builtin_bit_cast(unsigned short, a.lr[o]);
    p.be = g.momentum ? __builtin_bit_cast(unsigned short, a.beta[o]) : (unsigned short)0;
  }
  // window weight w(r, j) of target r, lag j: the lag gate, the gate of the source token t0 + r - j,
  // or 1; zero for targets past T
#pragma unroll
  for (int u = 0; u < 3; ++u) {
    p.gt[u] = 0;
    const int i = tid + NTB * u;
    const int r = i / g.e, j = i - r * g.e;
    if (r < CL && t0 + r < g.T) {
      if (g.gate_mode == GATE_LAG) {
        p.gt[u] = __builtin_bit_cast(unsigned short, a.gate[(rowbase + t0 + r) * g.e + j]);
      } else if (g.gate_mode == GATE_TOKEN) {
        if (t0 + r - j >= 0) p.gt[u] = __builtin_bit_cast(unsigned short, a.gate[rowbase + t0 + r - j]);
      } else {
        p.gt[u] = 0x3f80;
      }
    }
  }
}
__device__ __forceinline__ void gates_store(const ScalPf& p, const Geom& g, BwSm& sm) {
  const int tid = fresh_tid();
#pragma unroll
  for (int u = 0; u < 3; ++u) {
    const int i = tid + NTB * u;
    if (i < CL * g.e) {
      const int r = i / g.e, j = i - r * g.e;
      sm.Bd[r + HT - j][r] = __builtin_bit_cast(bf16, p.gt[u]);
    }
  }
}

// window weight of lag j for chunk target r (the chunk's staged band)
__device__ __forceinline__ float cw(const BwSm& sm, int r, int j) { return static_cast<float>(sm.Bd[r + HT - j][r]); }

// B'[u][t] = the coefficient of g_u in Z_{t-1}: B(u -> t - 1) = exp2(LB[t-1] - LB[u]) for u <= t - 1
// with momentum, [u == t - 1] without. Operand rows t (lane & 15), k slots natural over u.
template <bool MOM>
__device__ __forceinline__ bf16x8 gen_zcoef(const float* lb, int t, int q, int lane) {
  if constexpr (MOM) return gen_decay_to(lb, t, q, lane);
  const int gq = lane >> 4;
  bf16x8 f;
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = static_cast<bf16>(32 * q + 8 * gq + e == t - 1 ? 1.f : 0.f);
  return f;
}

// wave 0: the chunk's end coefficients (cgS, cgZ per target; the transition) from its scalars
__device__ __forceinline__ void chunk_end_scan(const Geom& g, const ScalPf& p, int t0, BwSm& sm) {
  const int lane = fresh_tid() & 63;
  // lane j holds target r = 63 - j (the chunk read backwards); targets past T are the identity
  const float al = __shfl(bf(p.al), 63 - lane, 64), et = __shfl(bf(p.et), 63 - lane, 64),
              be = __shfl(bf(p.be), 63 - lane, 64);
  const Tri x{al, -et * be, be};
  const Tri inc = wave_scan<false>(x, lane);
  Tri ex = tri_prev_lane(inc);
  if (lane == 0) ex = tri_id();
  const int r = 63 - lane;
  const bool real = t0 + r < g.T;
  sm.co[R_GS + r] = real ? ex.k - et * ex.a : 0.f;
  sm.co[R_GZ + r] = real ? ex.b : 0.f;
  if (lane == 63) { sm.co[R_TR] = inc.a; sm.co[R_TR + 1] = inc.k; sm.co[R_TR + 2] = inc.b; sm.co[R_TR + 3] = 0.f; }
}
// threads < 80: the per-source end coefficients from cgS / cgZ (needs chunk_end_scan's output)
__device__ __forceinline__ void chunk_end_sources(const Geom& g, BwSm& sm) {
  const int s = fresh_tid();
  if (s < SRC) {
    float cs = 0.f, cz = 0.f;
    for (int j = 0; j < g.e; ++j) {
      const int r = s - HT + j;
      if (r >= 0 && r < CL) {
        const float wgt = cw(sm, r, j);
        cs += wgt * sm.co[R_GS + r];
        cz += wgt * sm.co[R_GZ + r];
      }
    }
    sm.co[R_CS + s] = cs;
    sm.co[R_CZ + s] = cz;
  }
}

// wave 0: the chunk's prefix arrays: LA, LB (log2 prefix sums), eta, beta, and the coefficients of
// (S_c, Z_c) in S_{t-1} (At, Kt) and of Z_c in Z_{t-1} (B1)
__device__ __forceinline__ void chunk_prefix(const ScalPf& p, BwSm& sm) {
  const int lane = fresh_tid() & 63;
  const float al = bf(p.al), et = bf(p.et), be = bf(p.be);
  sm.la[lane] = wave_prefix_sum(fmaxf(__log2f(al), kLogFloor), lane);
  sm.lb[lane] = wave_prefix_sum(fmaxf(__log2f(be), kLogFloor), lane);
  sm.eta[lane] = et;
  sm.be[lane] = be;
  const Tri inc = wave_scan<true>(Tri{al, -et * be, be}, lane);
  Tri ex = tri_prev_lane(inc);
  if (lane == 0) ex = tri_id();
  sm.At[lane] = ex.a;
  sm.Kt[lane] = ex.k;
  sm.B1[lane] = ex.b;
}

// Sum over the 64 lanes, in every lane (DPP row sums, then the cross-row swaps).
__device__ __forceinline__ float wave_sum(float x) { return xsum_rows(row_sum16(x)); }

__device__ __forceinline__ unsigned pk(float a, float b) { return pack_bf16x2(a, b); }
// v stored at byte offset off (32-bit) from a uniform base: one store with a scalar base and a 32-bit
// vector offset instead of per-lane 64-bit address arithmetic
template <typename T>
__device__ __forceinline__ void st_at(T* base, uint32_t off, T v) {
  *reinterpret_cast<T*>(reinterpret_cast<unsigned char*>(base) + off) = v;
}
__device__ __forceinline__ float lo16(unsigned u) { return __builtin_bit_cast(float, u << 16); }
__device__ __forceinline__ float hi16(unsigned u) { return __builtin_bit_cast(float, u & 0xffff0000u); }

}  // namespace cpb

using namespace cpb;

template <bool MAPE, bool MOM>
__global__ __launch_bounds__(NTB) void k_cp_bwd(const Geom g, const BwdPtrs<bf16> a, const SegGeom sg,
                                                 const BwdSegPtrs p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  BwSm& sm = *reinterpret_cast<BwSm*>(smem_raw);
  const int tid = threadIdx.x, lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gq = lane >> 4, m = lane & 15;
  const int q4 = w & 3, hf = w >> 2;
  const int seg = blockIdx.x, bh = blockIdx.y;
  const int c_begin = seg * sg.G, c_end = min(g.nc, c_begin + sg.G);
  const int tok0 = c_begin * CL, tok1 = min(g.T, c_end * CL);
  const int H = g.H;
  const int tail0 = tok1 - H;   // the segment's last H tokens: partial results for the fixup
  const size_t rowbase = (size_t)bh * g.T;
  const size_t DD = (size_t)D * D;
  const uint32_t row_bytes = (uint32_t)g.T * (D * 2);
  const rsrc_t rk = make_rsrc(a.k + rowbase * D, row_bytes);
  const rsrc_t rv = make_rsrc(a.v + rowbase * D, row_bytes);
  const rsrc_t rq = make_rsrc(a.q + rowbase * D, row_bytes);
  const rsrc_t rdy = make_rsrc(a.dy + rowbase * D, row_bytes);
  const rsrc_t rdq = make_rsrc(a.dq + rowbase * D, row_bytes);

  bf16x8 sref[2];
  load_sref(a.S_ref + (size_t)bh * DD, q4, sref);
  // S_ref^T operand of dphi (waves 4-7, column tile q4): Bt[k = 16 q4 + m][i = 32 q + 8 gq + e]
  bf16x8 sreft[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const float* sr = a.S_ref + (size_t)bh * DD + (size_t)(32 * q + 8 * gq) * D + 16 * q4 + m;
    bf16x8 f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = static_cast<bf16>(sr[e * D]);
    sreft[q] = f;
  }

  // the band's entries off the window stay zero; its window entries are rewritten for every chunk
  for (int i = tid; i < SRC * PB / 2; i += NTB) reinterpret_cast<unsigned*>(&sm.Bd[0][0])[i] = 0u;
  __syncthreads();
  // ---------------------------------------------------------------- forward pass over the segment
  float xS[2][4], xZ[2][4];
  {
    const float* ss = p.seg_states + ((size_t)bh * sg.nseg + seg) * 2 * DD;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int off = (16 * q4 + 4 * gq + r) * D + 16 * (2 * hf + j) + m;
        xS[j][r] = ss[off];
        xZ[j][r] = MOM ? ss[DD + off] : 0.f;
      }
  }
  // per chunk of the segment: its chunk-start state (S_c^T, Z_c^T as bf16 [k][i], the LDS layout of
  // XS) and its coefficient record, kept in the workspace between the two passes
  unsigned char* xs_seg = reinterpret_cast<unsigned char*>(p.xsave) + ((size_t)bh * sg.nseg + seg) * sg.G * kXsBytes;
  {
    RowPf<WL_F> pf;
    ScalPf sp;
    rows_load<WL_F>(pf, rk, rv, rq, rdy, c_begin * CL, w);
    scal_load(sp, g, a, rowbase, c_begin * CL);
#pragma unroll 1
    for (int cc = 0; cc < c_end - c_begin; ++cc) {
      const int c = c_begin + cc;
      {
        CPB_FRESH_LANE
        const int t0 = c * CL;
        if (cc > 0) __syncthreads();
        rows_store<MAPE, WL_F>(pf, sm, g.map_deg, w);
        gates_store(sp, g, sm);
        const ScalPf spc = sp;
        if (c + 1 < c_end) {
          rows_load<WL_F>(pf, rk, rv, rq, rdy, t0 + CL, w);
          scal_load(sp, g, a, rowbase, t0 + CL);
        } else {
          pf = RowPf<WL_F>{};
          sp = ScalPf{};
        }
        __syncthreads();
        if (w == 0) chunk_end_scan(g, spc, t0, sm);
        // delta[s][i] for this wave's rows i (tiles of 16 sources)
        f32x4 dl[SRC / 16];
#pragma unroll
        for (int st = 0; st < SRC / 16; ++st) {
          dl[st] = zero4();
#pragma unroll
          for (int q = 0; q < 2; ++q) dl[st] = mma_bf16(frag_row_l(&sm.phi[0][0], PB, 16 * st, 32 * q, lane), sref[q], dl[st]);
          const s16x4 vt = tr4_l(&sm.vd[0][0], PB, 16 * st, 16 * q4, lane);
#pragma unroll
          for (int r = 0; r < 4; ++r) dl[st][r] -= bf((unsigned short)vt[r]);
        }
        __syncthreads();
        chunk_end_sources(g, sm);
        __syncthreads();
        unsigned char* xsc = xs_seg + (size_t)cc * kXsBytes;
        if (tid < REC) reinterpret_cast<float*>(xsc + kXsStates)[tid] = sm.co[tid];
        f32x4 U[2], V[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) { U[j] = zero4(); V[j] = zero4(); }
#pragma unroll
        for (int q = 0; q < 3; ++q) {
          const float4 chi = *reinterpret_cast<const float4*>(&sm.co[R_CS + 32 * q + 4 * gq]);
          const float4 zhi = *reinterpret_cast<const float4*>(&sm.co[R_CZ + 32 * q + 4 * gq]);
          float4 clo = make_float4(0.f, 0.f, 0.f, 0.f), zlo = clo;
          if (q < 2) {
            clo = *reinterpret_cast<const float4*>(&sm.co[R_CS + 32 * q + 16 + 4 * gq]);
            zlo = *reinterpret_cast<const float4*>(&sm.co[R_CZ + 32 * q + 16 + 4 * gq]);
          }
          const f32x4 lo = q < 2 ? dl[2 * q + 1] : zero4();
          const bf16x8 fs = pack_frag_scaled(dl[2 * q], lo, chi, clo);
          const bf16x8 fz = pack_frag_scaled(dl[2 * q], lo, zhi, zlo);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int kt = 2 * hf + j;
            const bf16x8 fb = q < 2 ? tr_pair_l<true>(&sm.phi[0][0], PB, q, 16 * kt, lane) : tr_pair_l<false>(&sm.phi[0][0], PB, q, 16 * kt, lane);
            U[j] = mma_bf16(fs, fb, U[j]);
            V[j] = mma_bf16(fz, fb, V[j]);
          }
        }
        const float ta = sm.co[R_TR], tk = sm.co[R_TR + 1], tb = sm.co[R_TR + 2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int kt = 2 * hf + j;
          const size_t o = ((size_t)(16 * kt + m) * D + 16 * q4 + 4 * gq) * 2;
          *reinterpret_cast<uint2*>(xsc + o) = make_uint2(pk(xS[j][0], xS[j][1]), pk(xS[j][2], xS[j][3]));
          *reinterpret_cast<uint2*>(xsc + DD * 2 + o) = make_uint2(pk(xZ[j][0], xZ[j][1]), pk(xZ[j][2], xZ[j][3]));
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float sn = ta * xS[j][r] + tk * xZ[j][r] + U[j][r];
            xZ[j][r] = MOM ? tb * xZ[j][r] + V[j][r] : 0.f;
            xS[j][r] = sn;
          }
        }
      }
    }
  }

  // ---------------------------------------------------------------- reverse pass
  float lS[2][4], lZ[2][4];
  {
    const float* sa = p.seg_adj + ((size_t)bh * sg.nseg + seg) * 2 * DD;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int off = (16 * q4 + 4 * gq + r) * D + 16 * (2 * hf + j) + m;
        lS[j][r] = sa[off];
        lZ[j][r] = MOM ? sa[DD + off] : 0.f;
      }
  }
  float cdv[4], cdk[4];     // halo partials (dv, dphi) of rows 0 .. 15 of the chunk just done
#pragma unroll
  for (int r = 0; r < 4; ++r) { cdv[r] = 0.f; cdk[r] = 0.f; }
  f32x4 dsr[4];             // dS_ref partial (waves 0-3: rows 16 q4 .., column tiles kt)
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) dsr[kt] = zero4();
  // Gram columns 82 .. 103 stay zero
  for (int i = tid; i < CL * (MP - 82); i += NTB) sm.Mt[i / (MP - 82)][82 + i % (MP - 82)] = static_cast<bf16>(0.f);

  RowPf<WL_R> pf;
  ScalPf sp;
  rows_load<WL_R>(pf, rk, rv, rq, rdy, (c_end - 1) * CL, w);
  scal_load(sp, g, a, rowbase, (c_end - 1) * CL);
#pragma unroll 1
  for (int cr = c_end - c_begin - 1; cr >= 0; --cr) {
    CPB_FRESH_LANE
    const int c = c_begin + cr;
    const int t0 = c * CL;
    const unsigned char* xsc = xs_seg + (size_t)cr * kXsBytes;
    // this wave's slice of X_c (for the Grams) and the record
    unsigned xc[8];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int kt = 2 * hf + j;
      const size_t o = ((size_t)(16 * kt + m) * D + 16 * q4 + 4 * gq) * 2;
      const uint2 a0 = *reinterpret_cast<const uint2*>(xsc + o);
      const uint2 a1 = *reinterpret_cast<const uint2*>(xsc + DD * 2 + o);
      xc[4 * j + 0] = a0.x; xc[4 * j + 1] = a0.y; xc[4 * j + 2] = a1.x; xc[4 * j + 3] = a1.y;
    }
    const float rc = tid < REC ? reinterpret_cast<const float*>(xsc + kXsStates)[tid] : 0.f;
    const bool seg_last = c == c_end - 1, seg_first = c == c_begin;
    // ---- R0: stage the chunk
    __syncthreads();
    rows_store<MAPE, WL_R>(pf, sm, g.map_deg, w);
    gates_store(sp, g, sm);
    if (w == 0) chunk_prefix(sp, sm);
    if (tid < REC) sm.co[tid] = rc;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int kt = 2 * hf + j;
      bf16* xs = &sm.XS[0][16 * kt + m][16 * q4 + 4 * gq];
      bf16* xz = &sm.XS[1][16 * kt + m][16 * q4 + 4 * gq];
      *reinterpret_cast<uint2*>(xs) = make_uint2(xc[4 * j + 0], xc[4 * j + 1]);
      *reinterpret_cast<uint2*>(xz) = make_uint2(xc[4 * j + 2], xc[4 * j + 3]);
      *reinterpret_cast<uint2*>(&sm.XL[0][16 * kt + m][16 * q4 + 4 * gq]) =
          make_uint2(pk(lS[j][0], lS[j][1]), pk(lS[j][2], lS[j][3]));
      *reinterpret_cast<uint2*>(&sm.XL[1][16 * kt + m][16 * q4 + 4 * gq]) =
          make_uint2(pk(lZ[j][0], lZ[j][1]), pk(lZ[j][2], lZ[j][3]));
    }
    // the four state-adjoint Grams over this wave's slice (X_c from its bf16 copy)
    {
      float gss = 0.f, gsz = 0.f, gzs = 0.f, gzz = 0.f;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float s4[4] = {lo16(xc[4 * j]), hi16(xc[4 * j]), lo16(xc[4 * j + 1]), hi16(xc[4 * j + 1])};
        const float z4[4] = {lo16(xc[4 * j + 2]), hi16(xc[4 * j + 2]), lo16(xc[4 * j + 3]),
                             hi16(xc[4 * j + 3])};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          gss += lS[j][r] * s4[r]; gsz += lS[j][r] * z4[r];
          gzs += lZ[j][r] * s4[r]; gzz += lZ[j][r] * z4[r];
        }
      }
      gss = wave_sum(gss); gsz = wave_sum(gsz); gzs = wave_sum(gzs); gzz = wave_sum(gzz);
      if (lane == 0) { sm.gram[w][0] = gss; sm.gram[w][1] = gsz; sm.gram[w][2] = gzs; sm.gram[w][3] = gzz; }
    }
    __syncthreads();

    // ---- R1: delta (in place of v), C'
    {
      CPB_FRESH_LANE
      const int st0 = hf == 0 ? 0 : 3, nst = hf == 0 ? 3 : 2;
      for (int u = 0; u < nst; ++u) {
        const int st = st0 + u;
        f32x4 acc = zero4();
#pragma unroll
        for (int q = 0; q < 2; ++q) acc = mma_bf16(sref[q], frag_row_l(&sm.phi[0][0], PB, 16 * st, 32 * q, lane), acc);
        bf16* pv = &sm.vd[16 * st + m][16 * q4 + 4 * gq];
        const float4 vv = lds_bf16x4(pv);
        store4<bf16>(pv, acc[0] - vv.x, acc[1] - vv.y, acc[2] - vv.z, acc[3] - vv.w);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int tt = 2 * hf + j;
        f32x4 acc = zero4();
#pragma unroll
        for (int q = 0; q < 2; ++q)
          acc = mma_bf16(gen_beta_eta<MOM>(sm.lb, sm.eta, 16 * q4 + m, q, lane), gen_decay_to(sm.la, 16 * tt + m, q, lane), acc);
#pragma unroll
        for (int r = 0; r < 4; ++r) sm.Cb[16 * q4 + 4 * gq + r][16 * tt + m] = static_cast<bf16>(acc[r]);
      }
    }
    __syncthreads();

    // ---- R2: t-phase (waves 0-3) | end terms of ddelta / dphi (waves 4-7)
    if (hf == 0) {
      CPB_FRESH_LANE
      const int tt = q4;
      const int t = 16 * tt + m;
      // C' as the k-major operand over the targets r (lane row t): shared by every source tile
      const bf16x8 fcb0 = frag_tr_l(&sm.Cb[0][0], PB, 16 * tt, 0, lane);
      const bf16x8 fcb1 = frag_tr_l(&sm.Cb[0][0], PB, 16 * tt, 32, lane);
      f32x4 Rr[SRC / 16];
#pragma unroll
      for (int st = 0; st < SRC / 16; ++st) {
        f32x4 kq = zero4(), dd = zero4(), wy = zero4();
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          kq = mma_bf16(frag_row_l(&sm.phi[0][0], PB, 16 * st, 32 * q, lane), frag_row_l(&sm.psi[0][0], PB, 16 * tt, 32 * q, lane), kq);
          dd = mma_bf16(frag_row_l(&sm.vd[0][0], PB, 16 * st, 32 * q, lane), frag_row_l(&sm.dy[0][0], PB, 16 * tt, 32 * q, lane), dd);
        }
        // Wy[s][t] = sum_r Band[s][r] C'[r][t]: the band of source tile st meets targets
        // 16 st - 16 .. 16 st + e - 2 only (e <= 17): k half 0 for st <= 2, half 1 for st >= 2
        if (st <= 2) wy = mma_bf16(frag_row_l(&sm.Bd[0][0], PB, 16 * st, 0, lane), fcb0, wy);
        if (st >= 2) wy = mma_bf16(frag_row_l(&sm.Bd[0][0], PB, 16 * st, 32, lane), fcb1, wy);
        float qv[4], rv_[4], mv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          qv[r] = kq[r] * wy[r];
          rv_[r] = dd[r] * wy[r];
          mv[r] = kq[r] * dd[r];
          Rr[st][r] = rv_[r];
        }
        store4<bf16>(&sm.Qt[t][16 * st + 4 * gq], qv[0], qv[1], qv[2], qv[3]);
        store4<bf16>(&sm.Rt[t][16 * st + 4 * gq], rv_[0], rv_[1], rv_[2], rv_[3]);
        store4<bf16>(&sm.Mt[t][16 * st + 4 * gq], mv[0], mv[1], mv[2], mv[3]);
      }
      // dpsi^T[k][t]: intra-chunk sources, then the chunk-start state
      const bf16x8 fr0 = pack_frag(Rr[0], Rr[1]), fr1 = pack_frag(Rr[2], Rr[3]), fr2 = pack_frag(Rr[4], zero4());
      const float At = sm.At[t], Kt = sm.Kt[t];
      float fS = 0.f, fZ = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        f32x4 di = zero4(), ds = zero4(), dz = zero4();
        di = mma_bf16(tr_pair_l<true>(&sm.phi[0][0], PB, 0, 16 * kt, lane), fr0, di);
        di = mma_bf16(tr_pair_l<true>(&sm.phi[0][0], PB, 1, 16 * kt, lane), fr1, di);
        di = mma_bf16(tr_pair_l<false>(&sm.phi[0][0], PB, 2, 16 * kt, lane), fr2, di);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const bf16x8 fdy = frag_row_l(&sm.dy[0][0], PB, 16 * tt, 32 * q, lane);
          ds = mma_bf16(frag_row_l(&sm.XS[0][0][0], PB, 16 * kt, 32 * q, lane), fdy, ds);
          dz = mma_bf16(frag_row_l(&sm.XS[1][0][0], PB, 16 * kt, 32 * q, lane), fdy, dz);
        }
        const float4 ps = lds_bf16x4(&sm.psi[t][16 * kt + 4 * gq]);
        fS += ps.x * ds[0] + ps.y * ds[1] + ps.z * ds[2] + ps.w * ds[3];
        fZ += ps.x * dz[0] + ps.y * dz[1] + ps.z * dz[2] + ps.w * dz[3];
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = di[r] + At * ds[r] + Kt * dz[r];
        if constexpr (MAPE) {
          const u32x2v raw = bld8(rq, (uint32_t)(((t0 + t) * D + 16 * kt + 4 * gq) * 2));
          o[0] *= poly_map_grad(lo16(raw[0]), g.map_deg); o[1] *= poly_map_grad(hi16(raw[0]), g.map_deg);
          o[2] *= poly_map_grad(lo16(raw[1]), g.map_deg); o[3] *= poly_map_grad(hi16(raw[1]), g.map_deg);
        }
        u32x2v out;
        out[0] = pk(o[0], o[1]);
        out[1] = pk(o[2], o[3]);
        bst8(rdq, (uint32_t)(((t0 + t) * D + 16 * kt + 4 * gq) * 2), out);
      }
      fS = xsum_rows(fS);
      fZ = xsum_rows(fZ);
      if (gq == 0) {
        sm.Mt[t][SRC] = static_cast<bf16>(fS);
        sm.Mt[t][SRC + 1] = static_cast<bf16>(fZ);
      }
    } else {
      CPB_FRESH_LANE
      const int ct = q4;
#pragma unroll
      for (int st = 0; st < SRC / 16; ++st) {
        f32x4 es = zero4(), ez = zero4(), fs = zero4(), fz = zero4();
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const bf16x8 fp = frag_row_l(&sm.phi[0][0], PB, 16 * st, 32 * q, lane);
          es = mma_bf16(fp, frag_tr_l(&sm.XL[0][0][0], PB, 16 * ct, 32 * q, lane), es);
          ez = mma_bf16(fp, frag_tr_l(&sm.XL[1][0][0], PB, 16 * ct, 32 * q, lane), ez);
          const bf16x8 fd = frag_row_l(&sm.vd[0][0], PB, 16 * st, 32 * q, lane);
          fs = mma_bf16(fd, frag_row_l(&sm.XL[0][0][0], PB, 16 * ct, 32 * q, lane), fs);
          fz = mma_bf16(fd, frag_row_l(&sm.XL[1][0][0], PB, 16 * ct, 32 * q, lane), fz);
        }
        const s16x4 dt = tr4_l(&sm.vd[0][0], PB, 16 * st, 16 * ct, lane);
        const float4 cs4 = *reinterpret_cast<const float4*>(&sm.co[R_CS + 16 * st + 4 * gq]);
        const float4 cz4 = *reinterpret_cast<const float4*>(&sm.co[R_CZ + 16 * st + 4 * gq]);
        const float csv[4] = {cs4.x, cs4.y, cs4.z, cs4.w}, czv[4] = {cz4.x, cz4.y, cz4.z, cz4.w};
        float ev[4], fv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float dv = bf((unsigned short)dt[r]);
          const float hs = row_sum16(dv * es[r]), hz = row_sum16(dv * ez[r]);
          if (m == 0) { sm.hp[0][ct][16 * st + 4 * gq + r] = hs; sm.hp[1][ct][16 * st + 4 * gq + r] = hz; }
          ev[r] = csv[r] * es[r] + czv[r] * ez[r];
          fv[r] = csv[r] * fs[r] + czv[r] * fz[r];
        }
        sm.ed[ct][st][0][lane] = pk(ev[0], ev[1]);
        sm.ed[ct][st][1][lane] = pk(ev[2], ev[3]);
        sm.ef[ct][st][0][lane] = pk(fv[0], fv[1]);
        sm.ef[ct][st][1][lane] = pk(fv[2], fv[3]);
      }
    }
    __syncthreads();

    // ---- R3: ddelta, dv (waves 4-7) | scalar gradients (waves 0-3)
    if (hf == 1) {
      CPB_FRESH_LANE
      const int ct = q4;
      float cin[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) cin[r] = cdv[r];
#pragma unroll
      for (int st = 0; st < SRC / 16; ++st) {
        f32x4 acc;
        {
          const unsigned e0 = sm.ed[ct][st][0][lane], e1 = sm.ed[ct][st][1][lane];
          acc[0] = lo16(e0); acc[1] = hi16(e0); acc[2] = lo16(e1); acc[3] = hi16(e1);
        }
#pragma unroll
        for (int q = 0; q < 2; ++q)
          acc = mma_bf16(frag_tr_l(&sm.Qt[0][0], QP, 16 * st, 32 * q, lane),
                         frag_tr_l(&sm.dy[0][0], PB, 16 * ct, 32 * q, lane), acc);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int s = 16 * st + 4 * gq + r;
          const float dd = acc[r];   // ddelta
          sm.vd[s][16 * ct + m] = static_cast<bf16>(dd);
          const int pp = t0 - HT + s, col = 16 * ct + m;
          if (st == 0) {   // halo rows: partial for the previous chunk (or the previous segment)
            if (seg_first) {
              if (seg > 0 && s >= HT - H)
                st_at(part_row(p.halo_part, bh, sg.nseg, seg, H), (uint32_t)(((s - (HT - H)) * (2 * D) + col) * 4), -dd);
            } else {
              cdv[r] = -dd;
            }
          } else if (pp < g.T) {
            float val = -dd + (st == SRC / 16 - 1 && !seg_last ? cin[r] : 0.f);
            if (pp >= tail0)
              st_at(part_row(p.tail_part, bh, sg.nseg, seg, H), (uint32_t)(((pp - tail0) * (2 * D) + col) * 4), val);
            else
              st_at(a.dv + rowbase * D, (uint32_t)((pp * D + col) * 2), static_cast<bf16>(val));
          }
        }
      }
    } else {
      CPB_FRESH_LANE
      const int tt = q4;
      float al[4] = {0.f, 0.f, 0.f, 0.f}, ea[4] = {0.f, 0.f, 0.f, 0.f}, eb[4] = {0.f, 0.f, 0.f, 0.f},
            bt[4] = {0.f, 0.f, 0.f, 0.f};
      const float gSS = sm.gram[0][0] + sm.gram[1][0] + sm.gram[2][0] + sm.gram[3][0] + sm.gram[4][0] + sm.gram[5][0] +
                        sm.gram[6][0] + sm.gram[7][0];
      const float gSZ = sm.gram[0][1] + sm.gram[1][1] + sm.gram[2][1] + sm.gram[3][1] + sm.gram[4][1] + sm.gram[5][1] +
                        sm.gram[6][1] + sm.gram[7][1];
      const float gZS = sm.gram[0][2] + sm.gram[1][2] + sm.gram[2][2] + sm.gram[3][2] + sm.gram[4][2] + sm.gram[5][2] +
                        sm.gram[6][2] + sm.gram[7][2];
      const float gZZ = sm.gram[0][3] + sm.gram[1][3] + sm.gram[2][3] + sm.gram[3][3] + sm.gram[4][3] + sm.gram[5][3] +
                        sm.gram[6][3] + sm.gram[7][3];
      // adjoint-coefficient operands (rows t = 16 tt + m, k = q natural): Am (decay), Km (C'); the
      // state-coefficient operands over the targets r (rows t): C'^T (of G_s in S_{t-1} through the
      // window: Wy = Band C'), B'^T (in Z_{t-1}: Wzy = Band B')
      bf16x8 fam[2], fzT[2];
      {
        const int t = 16 * tt + m;
        const float lat = sm.la[t];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int qq = 32 * q + 8 * gq + e;
            const float x = __builtin_amdgcn_exp2f(sm.la[qq > 0 ? qq - 1 : 0] - lat);
            fam[q][e] = static_cast<bf16>(qq > t ? x : 0.f);
          }
          fzT[q] = gen_zcoef<MOM>(sm.lb, t, q, lane);
        }
      }
      // per target row r of this lane: the end terms' coefficients (A(t -> 63); cgS, cgZ from the record)
      float aend[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) aend[r] = __builtin_amdgcn_exp2f(sm.la[CL - 1] - sm.la[16 * tt + 4 * gq + r]);
      // state bases s' = 16 sp2 + m: the products G_s (s' < 80), then S_c (80), Z_c (81)
#pragma unroll 1
      for (int sp2 = 0; sp2 < SRC / 16; ++sp2) {
        f32x4 ra = zero4(), rz = zero4(), wy = zero4(), wz = zero4();
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const bf16x8 fm = frag_tr_l(&sm.Mt[0][0], MP, 16 * sp2, 32 * q, lane);
          ra = mma_bf16(fam[q], fm, ra);
          rz = mma_bf16(frag_row_l(&sm.Cb[0][0], PB, 16 * tt, 32 * q, lane), fm, rz);
          const bf16x8 fb = frag_row_l(&sm.Bd[0][0], PB, 16 * sp2, 32 * q, lane);
          wy = mma_bf16(frag_tr_l(&sm.Cb[0][0], PB, 16 * tt, 32 * q, lane), fb, wy);
          wz = mma_bf16(fzT[q], fb, wz);
        }
        const int sq = 16 * sp2 + m;
        const float hs = sm.hp[0][0][sq] + sm.hp[0][1][sq] + sm.hp[0][2][sq] + sm.hp[0][3][sq];
        const float hz = sm.hp[1][0][sq] + sm.hp[1][1][sq] + sm.hp[1][2][sq] + sm.hp[1][3][sq];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 16 * tt + 4 * gq + r;
          const float Rs = ra[r] + aend[r] * hs;
          const float Rz = rz[r] + sm.co[R_GS + t] * hs + sm.co[R_GZ + t] * hz;
          al[r] += wy[r] * Rs;
          ea[r] += wz[r] * Rs;
          bt[r] += wz[r] * Rz;
          const int jb = t + HT - sq;   // band: the source of lag jb of target t
          const bool inb = jb >= 0 && jb < g.e;
          eb[r] += static_cast<float>(sm.Bd[sq][t]) * Rs;   // zero off the band
          if (inb && t0 + t < g.T) {
            const uint32_t o = (uint32_t)((t0 + t) * g.e + jb);
            if (g.gate_mode == GATE_LAG) st_at(a.dgate + rowbase * g.e, o * 2, static_cast<bf16>(Rz));
            else if (g.gate_mode == GATE_TOKEN) st_at(p.dw + rowbase * g.e, o * 4, Rz);
          }
        }
      }
      {   // s' = 80 (S_c: in S_{t-1} with At), 81 (Z_c: in S_{t-1} with Kt, in Z_{t-1} with B1)
        f32x4 ra = zero4(), rz = zero4();
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const bf16x8 fm = frag_tr_l(&sm.Mt[0][0], MP, SRC, 32 * q, lane);
          ra = mma_bf16(fam[q], fm, ra);
          rz = mma_bf16(frag_row_l(&sm.Cb[0][0], PB, 16 * tt, 32 * q, lane), fm, rz);
        }
        const bool bs = m == 0, bz = m == 1;
        const float hs = bs ? gSS : bz ? gSZ : 0.f;
        const float hz = bs ? gZS : bz ? gZZ : 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 16 * tt + 4 * gq + r;
          const float Rs = ra[r] + aend[r] * hs;
          const float Rz = rz[r] + sm.co[R_GS + t] * hs + sm.co[R_GZ + t] * hz;
          const float wy = bs ? sm.At[t] : bz ? sm.Kt[t] : 0.f;
          const float wz = bz ? sm.B1[t] : 0.f;
          al[r] += wy * Rs;
          ea[r] += wz * Rs;
          bt[r] += wz * Rz;
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float va = row_sum16(al[r]), vea = row_sum16(ea[r]), veb = row_sum16(eb[r]), vb = row_sum16(bt[r]);
        const int t = 16 * tt + 4 * gq + r;
        if (m == 0 && t0 + t < g.T) {
          const uint32_t o = (uint32_t)(t0 + t) * 2;
          st_at(a.ddecay + rowbase, o, static_cast<bf16>(va));
          st_at(a.dlr + rowbase, o, static_cast<bf16>(-(sm.be[t] * vea + veb)));
          if (MOM) st_at(a.dbeta + rowbase, o, static_cast<bf16>(vb));
        }
      }
    }
    __syncthreads();

    // ---- R4: dphi, dk (waves 4-7) | dS_ref partial (waves 0-3); the next chunk's rows in flight
    // (the last chunk clears the registers instead: the values just staged are dead from here on)
    if (c > c_begin) {
      rows_load<WL_R>(pf, rk, rv, rq, rdy, t0 - CL, w);
      scal_load(sp, g, a, rowbase, t0 - CL);
    } else {
      pf = RowPf<WL_R>{};
      sp = ScalPf{};
    }
    if (hf == 1) {
      CPB_FRESH_LANE
      const int ct = q4;
      const rsrc_t rkk = rk;
      float cin[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) cin[r] = cdk[r];
#pragma unroll
      for (int st = 0; st < SRC / 16; ++st) {
        f32x4 acc;
        {
          const unsigned e0 = sm.ef[ct][st][0][lane], e1 = sm.ef[ct][st][1][lane];
          acc[0] = lo16(e0); acc[1] = hi16(e0); acc[2] = lo16(e1); acc[3] = hi16(e1);
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          acc = mma_bf16(frag_tr_l(&sm.Rt[0][0], QP, 16 * st, 32 * q, lane),
                         frag_tr_l(&sm.psi[0][0], PB, 16 * ct, 32 * q, lane), acc);
          acc = mma_bf16(frag_row_l(&sm.vd[0][0], PB, 16 * st, 32 * q, lane), sreft[q], acc);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int s = 16 * st + 4 * gq + r;
          const float df = acc[r];
          const int pp = t0 - HT + s, col = 16 * ct + m;
          if (st == 0) {
            if (seg_first) {
              if (seg > 0 && s >= HT - H)
                st_at(part_row(p.halo_part, bh, sg.nseg, seg, H), (uint32_t)(((s - (HT - H)) * (2 * D) + D + col) * 4), df);
            } else {
              cdk[r] = df;
            }
          } else if (pp < g.T) {
            float val = df + (st == SRC / 16 - 1 && !seg_last ? cin[r] : 0.f);
            if (pp >= tail0) {
              st_at(part_row(p.tail_part, bh, sg.nseg, seg, H), (uint32_t)(((pp - tail0) * (2 * D) + D + col) * 4), val);
            } else {
              if constexpr (MAPE) val *= poly_map_grad(bf(bld2(rkk, (uint32_t)((pp * D + col) * 2))), g.map_deg);
              st_at(a.dk + rowbase * D, (uint32_t)((pp * D + col) * 2), static_cast<bf16>(val));
            }
          }
        }
      }
    } else {
      CPB_FRESH_LANE
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        f32x4 acc = zero4();
        acc = mma_bf16(tr_pair_l<true>(&sm.vd[0][0], PB, 0, 16 * q4, lane), tr_pair_l<true>(&sm.phi[0][0], PB, 0, 16 * kt, lane), acc);
        acc = mma_bf16(tr_pair_l<true>(&sm.vd[0][0], PB, 1, 16 * q4, lane), tr_pair_l<true>(&sm.phi[0][0], PB, 1, 16 * kt, lane), acc);
        acc = mma_bf16(tr_pair_l<false>(&sm.vd[0][0], PB, 2, 16 * q4, lane), tr_pair_l<false>(&sm.phi[0][0], PB, 2, 16 * kt, lane), acc);
#pragma unroll
        for (int r = 0; r < 4; ++r) dsr[kt][r] += acc[r];
      }
    }

    // ---- R5: the adjoint at the chunk start
    {
      CPB_FRESH_LANE
      const float ta = sm.co[R_TR], tk = sm.co[R_TR + 1], tb = sm.co[R_TR + 2];
      f32x4 dS[2], dZ[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) { dS[j] = zero4(); dZ[j] = zero4(); }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const bf16x8 fy = tr_pair_l<true>(&sm.dy[0][0], PB, q, 16 * q4, lane);
        const float4 ahi = *reinterpret_cast<const float4*>(&sm.At[32 * q + 4 * gq]);
        const float4 alo = *reinterpret_cast<const float4*>(&sm.At[32 * q + 16 + 4 * gq]);
        const float4 khi = *reinterpret_cast<const float4*>(&sm.Kt[32 * q + 4 * gq]);
        const float4 klo = *reinterpret_cast<const float4*>(&sm.Kt[32 * q + 16 + 4 * gq]);
        f32x4 yh, yl;
#pragma unroll
        for (int e = 0; e < 4; ++e) { yh[e] = static_cast<float>(fy[e]); yl[e] = static_cast<float>(fy[4 + e]); }
        const bf16x8 fa = pack_frag_scaled(yh, yl, ahi, alo);
        const bf16x8 fk = pack_frag_scaled(yh, yl, khi, klo);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const bf16x8 fp = tr_pair_l<true>(&sm.psi[0][0], PB, q, 16 * (2 * hf + j), lane);
          dS[j] = mma_bf16(fa, fp, dS[j]);
          dZ[j] = mma_bf16(fk, fp, dZ[j]);
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float ns = ta * lS[j][r] + dS[j][r];
          lZ[j][r] = MOM ? tk * lS[j][r] + tb * lZ[j][r] + dZ[j][r] : 0.f;
          lS[j][r] = ns;
        }
    }
  }

  // ---- segment results: dS0 / dZ0 (segment 0), the dS_ref partial
  if (seg == 0) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const size_t off = (size_t)bh * DD + (16 * q4 + 4 * gq + r) * D + 16 * (2 * hf + j) + m;
        a.dS0[off] = lS[j][r];
        if (MOM && a.dZ0) a.dZ0[off] = lZ[j][r];
      }
  }
  if (hf == 0) {
    float* dp = p.dsref_part + ((size_t)bh * sg.nseg + seg) * DD;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) dp[(16 * q4 + 4 * gq + r) * D + 16 * kt + m] = dsr[kt][r];
  }
}

template <bool OUTBUF>
__global__ __launch_bounds__(kThreads) void k_cp_fixup(const Geom g, const BwdPtrs<bf16> a, const SegGeom sg,
                                                        const BwdSegPtrs p, int reduce_dsref) {
  bwd_seg_fixup<bf16, 64, OUTBUF>(g, a, sg, p, reduce_dsref, blockIdx.x, blockIdx.y);
}

__global__ __launch_bounds__(kThreads) void k_cp_reduce_dsref(int nseg, const float* part, float* out) {
  const int bh = blockIdx.y;
  const int idx = blockIdx.x * kThreads + threadIdx.x;
  if (idx >= 64 * 64) return;
  float acc = 0.f;
  for (int s = 0; s < nseg; ++s) acc += part[((size_t)bh * nseg + s) * 64 * 64 + idx];
  out[(size_t)bh * 64 * 64 + idx] = acc;
}

bool chunk_bwd_supported(const Geom& g, const SegGeom& sg) {
  return g.DK == 64 && g.DV == 64 && g.Lc == CL && g.H <= HT && g.clamp_every == 0 && g.clamp_check == 0 &&
         !g.has_buf && g.flag == nullptr && sg.G >= 1;
}

// Workspace of k_cp_bwd: per chunk its start state (bf16) and coefficient record.
size_t chunk_bwd_xsave_bytes(const Geom& g, const SegGeom& sg) {
  return (size_t)g.BH * sg.nseg * sg.G * kXsBytes;
}

// g, sg: the forward's chunks (64 tokens) and segments. p.seg_adj must hold the adjoint at every
// segment end (k_bwd_seg_agg / k_bwd_seg_scan); p.tail_part / halo_part / dw / dsref_part are the
// backward workspace of the shared fixup.
hipError_t launch_chunk_bwd(const Geom& g, const BwdPtrs<bf16>& a, const SegGeom& sg, const BwdSegPtrs& p,
                            hipStream_t stream) {
  const bool mape = g.map_mode == MAP_ELEMENTWISE;
  const size_t smem = sizeof(BwSm);
  const void* fn = mape ? (g.momentum ? reinterpret_cast<const void*>(&k_cp_bwd<true, true>)
                                      : reinterpret_cast<const void*>(&k_cp_bwd<true, false>))
                        : (g.momentum ? reinterpret_cast<const void*>(&k_cp_bwd<false, true>)
                                      : reinterpret_cast<const void*>(&k_cp_bwd<false, false>));
  hipError_t err = set_dyn_smem(fn, smem);
  if (err != hipSuccess) return err;
  prof_name(KID_BWD_CHUNK, "k_cp_bwd");
  prof_begin(KID_BWD_CHUNK, stream);
  const dim3 grid(sg.nseg, g.BH);
  if (mape) {
    if (g.momentum) hipLaunchKernelGGL((k_cp_bwd<true, true>), grid, dim3(NTB), smem, stream, g, a, sg, p);
    else hipLaunchKernelGGL((k_cp_bwd<true, false>), grid, dim3(NTB), smem, stream, g, a, sg, p);
  } else {
    if (g.momentum) hipLaunchKernelGGL((k_cp_bwd<false, true>), grid, dim3(NTB), smem, stream, g, a, sg, p);
    else hipLaunchKernelGGL((k_cp_bwd<false, false>), grid, dim3(NTB), smem, stream, g, a, sg, p);
  }
  prof_end(KID_BWD_CHUNK, stream);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  const int fused_reduce = a.dbuf_out == nullptr;
  prof_name(KID_BWD_FIXUP, "k_cp_fixup");
  prof_begin(KID_BWD_FIXUP, stream);
  if (a.dbuf_out)
    hipLaunchKernelGGL((k_cp_fixup<true>), dim3(sg.nseg, g.BH), dim3(kThreads), 0, stream, g, a, sg, p, fused_reduce);
  else
    hipLaunchKernelGGL((k_cp_fixup<false>), dim3(sg.nseg, g.BH), dim3(kThreads), 0, stream, g, a, sg, p, fused_reduce);
  prof_end(KID_BWD_FIXUP, stream);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  if (fused_reduce) return hipSuccess;
  prof_begin(KID_REDUCE_DSREF, stream);
  hipLaunchKernelGGL(k_cp_reduce_dsref, dim3(64 * 64 / kThreads, g.BH), dim3(kThreads), 0, stream, sg.nseg,
                     (const float*)p.dsref_part, a.dS_ref);
  prof_end(KID_REDUCE_DSREF, stream);
  return hipGetLastError();
}

}  // namespace atlas
