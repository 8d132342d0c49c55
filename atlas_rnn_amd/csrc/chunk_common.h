// chunk_common.h - pieces of the chunk-parallel path (bf16 inputs, d_k = d_v = 64, window <= 17,
// no scan_chunk_len clamp, no carried buffer).
//
// The sequence of a head-batch row is cut into chunks of CL = 64 tokens and segments of SEGC = 4
// chunks. Every chunk is one independent workgroup: the state at its start is recomputed from the
// segment-start state (a short scan over segment aggregates) and the products of the segment's
// earlier chunks, as one matrix product whose k axis runs over those sources, with per-source
// coefficients from a scan of the 2 x 2 scalar transitions; nothing is stored per chunk.
//
// Notation (all per row; S, Z are d x d; g_t is the gated window sum at token t):
//   M_t = [[alpha_t, -eta_t beta_t], [0, beta_t]] maps (S, Z)_{t-1} to (S, Z)_t before g_t enters
//   as (-eta_t, 1) g_t (without momentum beta = 0, so Z_t = g_t). A product of such upper
//   triangular matrices is kept as a triple (a, k, b) = [[a, k], [0, b]].
//   Inside a chunk (local targets t = 0 .. 63): LA[t] = sum_{u <= t} log2 alpha_u, LB[t] likewise
//   for beta, so prod_{v = u+1 .. t} alpha_v = exp2(LA[t] - LA[u]) for t >= u (exponent <= 0: no
//   overflow; log2 is floored at kLogFloor so that a zero decay gives ~0 instead of NaN).
#pragma once

#include "mem_common.h"
#include "mem_params.h"
#include "seg_common.h"
#include "walk_common.h"

namespace atlas {
namespace cp {

constexpr int D = 64;               // head size (d_k = d_v)
constexpr int CL = 64;              // chunk length
constexpr int HT = 16;              // halo rows staged before a chunk's first token (window halo <= 16)
constexpr int SRC = CL + HT;        // source rows of a chunk
constexpr int NTH = 256;            // threads per workgroup
constexpr int NWV = NTH / 64;       // waves per workgroup
constexpr int SEGC = 4;             // chunks per segment
constexpr int SEGT = SEGC * CL;     // tokens per segment
constexpr int PD = D + 16;          // LDS pitch of 64-wide bf16 rows (elements): 160 bytes
constexpr int RMAX = SEGT;          // longest coefficient range (targets)
constexpr int SMAX = RMAX + 2 * CL; // per-source coefficient arrays, padded to whole 64-row blocks
constexpr float kLogFloor = -100.f;

struct Tri { float a, k, b; };
__device__ __forceinline__ Tri tri_id() { return Tri{1.f, 0.f, 1.f}; }
__device__ __forceinline__ Tri tri_mul(const Tri& L, const Tri& R) {
  return Tri{L.a * R.a, L.a * R.k + L.k * R.b, L.b * R.b};
}
// Lane moves on the VALU (DPP) for the wave-wide scans: `old` where the source lane is outside the
// pattern or its row is masked off. Controls: row_shr:n = 0x110 + n (within 16-lane rows),
// wave_shr:1 = 0x138, row_bcast:15 = 0x142 (lane 15 of a row to the next row), row_bcast:31 = 0x143
// (lane 31 to rows 2 and 3).
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_f(float old, float src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, src),
                                                               CTRL, ROWS, 0xf, false));
}
template <int CTRL, int ROWS>
__device__ __forceinline__ Tri dpp_tri(const Tri& x) {
  return Tri{dpp_f<CTRL, ROWS>(1.f, x.a), dpp_f<CTRL, ROWS>(0.f, x.k), dpp_f<CTRL, ROWS>(1.f, x.b)};
}
// The previous lane's value (lane 0: the identity).
__device__ __forceinline__ Tri tri_prev_lane(const Tri& x) { return dpp_tri<0x138, 0xf>(x); }

// Inclusive scan over the 64 lanes of a wave (row shifts 1, 2, 4, 8, then the row broadcasts).
// LATER_LEFT: lane j gets X_j X_{j-1} ... X_0 (the product of a forward recurrence); otherwise
// X_0 X_1 ... X_j.
template <bool LATER_LEFT>
__device__ __forceinline__ Tri wave_scan(Tri v, int lane) {
  (void)lane;
#define ATLAS_TRI_STEP(C, R)                         \
  {                                                  \
    const Tri u = dpp_tri<C, R>(v);                  \
    v = LATER_LEFT ? tri_mul(v, u) : tri_mul(u, v);  \
  }
  ATLAS_TRI_STEP(0x111, 0xf)
  ATLAS_TRI_STEP(0x112, 0xf)
  ATLAS_TRI_STEP(0x114, 0xf)
  ATLAS_TRI_STEP(0x118, 0xf)
  ATLAS_TRI_STEP(0x142, 0xa)
  ATLAS_TRI_STEP(0x143, 0xc)
#undef ATLAS_TRI_STEP
  return v;
}

// Inclusive sum over the 64 lanes of a wave.
__device__ __forceinline__ float wave_prefix_sum(float v, int lane) {
  (void)lane;
  v += dpp_f<0x111, 0xf>(0.f, v);
  v += dpp_f<0x112, 0xf>(0.f, v);
  v += dpp_f<0x114, 0xf>(0.f, v);
  v += dpp_f<0x118, 0xf>(0.f, v);
  v += dpp_f<0x142, 0xa>(0.f, v);
  v += dpp_f<0x143, 0xc>(0.f, v);
  return v;
}

__device__ __forceinline__ float bf(unsigned short h) { return __builtin_bit_cast(float, (unsigned)h << 16); }

// Coefficients of a range of targets [ta, ta + n) (n <= RMAX) on the state after token ta + n - 1:
//   cgS[r - ta], cgZ[r - ta]: of g_r in S_{ta+n-1} and Z_{ta+n-1};
//   cs[i], cz[i]: of the source product G_s, s = ta - HT + i, through the window terms whose
//                 targets lie in the range (zero past the range's sources, up to SMAX);
//   trans: (a, k, b) of (S, Z)_{ta-1}: S_{ta+n-1} = a S_{ta-1} + k Z_{ta-1} + ..., Z_... = b Z_{ta-1} + ...
struct RangeSm {
  float cgS[RMAX], cgZ[RMAX];
  alignas(16) float cs[SMAX];
  alignas(16) float cz[SMAX];
  Tri tot[NWV];
  Tri trans;
};

// Scalars of token r of a row (bf16 inputs); tokens outside [0, T) give the identity transition.
struct TokScal { float al, et, be; };
__device__ __forceinline__ TokScal tok_scalars(const Geom& g, const bf16* decay, const bf16* lr, const bf16* beta,
                                               size_t rowbase, int r) {
  TokScal s{1.f, 0.f, 1.f};
  if (r >= 0 && r < g.T) {
    s.al = static_cast<float>(decay[rowbase + r]);
    s.et = static_cast<float>(lr[rowbase + r]);
    s.be = g.momentum ? static_cast<float>(beta[rowbase + r]) : 0.f;
  }
  return s;
}

// Window weight of lag j for target r (token index), given the staged gates: lag gates
// wl[(r - r0) * e + j] for targets from r0, token gates ug[s - s0] for sources from s0.
__device__ __forceinline__ float win_w(const Geom& g, const float* wl, int r0, const float* ug, int s0, int r, int j) {
  if (g.gate_mode == GATE_LAG) return wl[(r - r0) * g.e + j];
  if (g.gate_mode == GATE_TOKEN) return ug[r - j - s0];
  return 1.f;
}

// Scalars of the token thread tid holds in range_coefs: r = ta + n - 1 - tid (the range read
// backwards), the identity past the range. Loaded by the caller early (one round trip with its
// other loads).
__device__ __forceinline__ TokScal range_scalars(const Geom& g, const bf16* decay, const bf16* lr, const bf16* beta,
                                                 size_t rowbase, int ta, int n) {
  const int j = threadIdx.x;
  TokScal sc{1.f, 0.f, 1.f};
  if (j < n) sc = tok_scalars(g, decay, lr, beta, rowbase, ta + n - 1 - j);
  return sc;
}

// Every thread of the workgroup calls this (barriers inside), with its range_scalars. The gates of
// the range must be staged: lag wl[(r - ta) * e + j] for r in [ta, ta + n), token
// ug[s - (ta - HT)] for the sources.
__device__ __forceinline__ void range_coefs(const Geom& g, const TokScal& sc, int ta, int n, RangeSm& rs,
                                            const float* wl, const float* ug) {
  const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
  const int j = tid;
  const int r = ta + n - 1 - j;
  const bool in = j < n;
  const Tri x{sc.al, -sc.et * sc.be, sc.be};
  // X_{n-1} X_{n-2} ... : earlier j on the left
  Tri v = wave_scan<false>(x, lane);
  if (lane == 63) rs.tot[w] = v;
  __syncthreads();
  Tri pre = tri_id();
  for (int u = 0; u < w; ++u) pre = tri_mul(pre, rs.tot[u]);
  v = tri_mul(pre, v);
  Tri ex = tri_prev_lane(v);
  if (lane == 0) ex = pre;
  if (tid == 0) {
    Tri all = tri_id();
    for (int u = 0; u < NWV; ++u) all = tri_mul(all, rs.tot[u]);
    rs.trans = all;
  }
  if (in) {
    const bool real = r < g.T;
    rs.cgS[r - ta] = real ? ex.k - sc.et * ex.a : 0.f;
    rs.cgZ[r - ta] = real ? ex.b : 0.f;
  }
  __syncthreads();
  // per source: the window terms whose targets lie in the range
  const int s0 = ta - HT;
  for (int i = tid; i < SMAX; i += NTH) {
    const int s = s0 + i;
    float cs = 0.f, cz = 0.f;
    if (i < n + HT) {
      for (int jj = 0; jj < g.e; ++jj) {
        const int rr = s + jj;
        if (rr >= ta && rr < ta + n) {
          const float wgt = win_w(g, wl, ta, ug, s0, rr, jj);
          cs += wgt * rs.cgS[rr - ta];
          cz += wgt * rs.cgZ[rr - ta];
        }
      }
    }
    rs.cs[i] = cs;
    rs.cz[i] = cz;
  }
}

// Stage the gates of targets [r0, r0 + n) (lag) or of sources [r0 - HT, r0 + n) (token) as fp32.
__device__ __forceinline__ void stage_gates(const Geom& g, const bf16* gate, size_t rowbase, int r0, int n, float* wl,
                                            float* ug) {
  const int tid = threadIdx.x;
  if (g.gate_mode == GATE_LAG) {
    const int cnt = n * g.e;
    for (int i = tid; i < cnt; i += NTH) {
      const int r = r0 + i / g.e;
      wl[i] = (r >= 0 && r < g.T) ? static_cast<float>(gate[(rowbase + r) * g.e + i % g.e]) : 0.f;
    }
  } else if (g.gate_mode == GATE_TOKEN) {
    for (int i = tid; i < n + HT; i += NTH) {
      const int s = r0 - HT + i;
      ug[i] = (s >= 0 && s < g.T) ? static_cast<float>(gate[rowbase + s]) : 0.f;
    }
  }
}

// S_ref rows 16 it .. +15 as an MFMA operand (k = 32 q + 8 gq + e, natural order).
__device__ __forceinline__ void load_sref(const float* S_ref_row, int it, bf16x8 (&f)[2]) {
  const int lane = lane_id(), gq = lane >> 4, m = lane & 15;
  const float* sr = S_ref_row + (size_t)(16 * it + m) * D;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const float4 x0 = *reinterpret_cast<const float4*>(sr + 32 * q + 8 * gq);
    const float4 x1 = *reinterpret_cast<const float4*>(sr + 32 * q + 8 * gq + 4);
    bf16x8 v;
    v[0] = static_cast<bf16>(x0.x); v[1] = static_cast<bf16>(x0.y); v[2] = static_cast<bf16>(x0.z);
    v[3] = static_cast<bf16>(x0.w); v[4] = static_cast<bf16>(x1.x); v[5] = static_cast<bf16>(x1.y);
    v[6] = static_cast<bf16>(x1.z); v[7] = static_cast<bf16>(x1.w);
    f[q] = v;
  }
}

// Staging of 64 consecutive token rows [tb0, tb0 + 64) of a [T, 64] bf16 row tensor: thread tid
// moves the 16-byte vectors tid and tid + 256 (rows tid / 8 and tid / 8 + 32, column chunk tid % 8).
// Rows outside the tensor read as zeros (buffer range check).
struct Blk64 { u32x4v v[2]; };
__device__ __forceinline__ void blk_load(Blk64& b, rsrc_t r, int tb0) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int row = (tid >> 3) + 32 * u;
    b.v[u] = bld16(r, (uint32_t)((tb0 + row) * (D * 2) + (tid & 7) * 16));
  }
}
template <bool MAPE>
__device__ __forceinline__ void blk_store(const Blk64& b, bf16* lds, int deg) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int row = (tid >> 3) + 32 * u;
    u32x4v x = b.v[u];
    if constexpr (MAPE) x = map_bf16x8(x, deg);
    *reinterpret_cast<u32x4v*>(lds + row * PD + (tid & 7) * 8) = x;
  }
}

// Up to NB blocks of 64 source rows (phi and v) of a row, loaded into registers at once so that a
// workgroup pays one memory round trip for all of them.
template <int NB>
struct SrcBlocks { Blk64 p[NB], v[NB]; };
template <int NB>
__device__ __forceinline__ void src_load(SrcBlocks<NB>& sb, rsrc_t rk, rsrc_t rv, int s0, int nsrc) {
  const int nblk = (nsrc + CL - 1) / CL;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    // blocks past nblk are loaded from rows past the tensor (zeros) and never used
    const int tb0 = b < nblk ? s0 + CL * b : (1 << 24);
    blk_load(sb.p[b], rk, tb0);
    blk_load(sb.v[b], rv, tb0);
  }
}

// The state contribution of the sources [s0, s0 + nsrc) (s0 = ta - HT of a RangeSm) of a row:
//   Sacc[kt] += sum_s cs_s delta_s phi_s^T,  Zacc[kt] += sum_s cz_s delta_s phi_s^T,
// delta_s = S_ref phi_s - v_s; wave w owns the state rows i in [16 w, +16): Sacc[kt] holds
// S[16 w + 4 gq + r][16 kt + m]. The blocks (already in registers, src_load) pass through
// phib / vb (LDS, 64 rows each) one at a time; every thread calls this (barriers inside).
template <bool MAPE, int NB>
__device__ __forceinline__ void state_blocks(const SrcBlocks<NB>& sb, int nsrc, const RangeSm& rs,
                                             const bf16x8 (&sref)[2], bf16* phib, bf16* vb, f32x4 (&Sacc)[4],
                                             f32x4 (&Zacc)[4], int deg) {
  const int lane = lane_id(), w = wave_id(), gq = lane >> 4;
  const int nblk = (nsrc + CL - 1) / CL;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (b < nblk) {   // workgroup-uniform
      if (b > 0) __syncthreads();   // the previous block's products are done with phib / vb
      blk_store<MAPE>(sb.p[b], phib, deg);
      blk_store<false>(sb.v[b], vb, deg);
      __syncthreads();
      const int i0 = CL * b;   // first source index of the block in rs.cs
      // delta[s][i] for the block's 64 sources (tiles st) and this wave's 16 rows i
      f32x4 dl[4];
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        dl[st] = zero4();
#pragma unroll
        for (int q = 0; q < 2; ++q) dl[st] = mma_bf16(frag_row(phib, PD, 16 * st, 32 * q), sref[q], dl[st]);
        const s16x4 vt = tr4(vb, PD, 16 * st, 16 * w);
#pragma unroll
        for (int r = 0; r < 4; ++r) dl[st][r] -= bf((unsigned short)vt[r]);
      }
      f32x4 sa[4], za[4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) { sa[kt] = zero4(); za[kt] = zero4(); }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const float4 chi = *reinterpret_cast<const float4*>(&rs.cs[i0 + 32 * q + 4 * gq]);
        const float4 clo = *reinterpret_cast<const float4*>(&rs.cs[i0 + 32 * q + 16 + 4 * gq]);
        const float4 zhi = *reinterpret_cast<const float4*>(&rs.cz[i0 + 32 * q + 4 * gq]);
        const float4 zlo = *reinterpret_cast<const float4*>(&rs.cz[i0 + 32 * q + 16 + 4 * gq]);
        const bf16x8 fs = pack_frag_scaled(dl[2 * q], dl[2 * q + 1], chi, clo);
        const bf16x8 fz = pack_frag_scaled(dl[2 * q], dl[2 * q + 1], zhi, zlo);
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          const bf16x8 fb = tr_pair<true>(phib, PD, q, 16 * kt);
          sa[kt] = mma_bf16(fs, fb, sa[kt]);
          za[kt] = mma_bf16(fz, fb, za[kt]);
        }
      }
      // block sums added outside the MFMA chain (the accumulators read after this branch are
      // never an MFMA's destination inside it)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) { Sacc[kt][r] += sa[kt][r]; Zacc[kt][r] += za[kt][r]; }
    }
  }
}

// Operand generators (row = lane & 15 of the tile, k slots natural: k = 32 q + 8 gq + e; lane passed in).
// B_eta[r][u] = -eta_u B(r -> u) for u >= r (r, u chunk-local targets).
template <bool MOM>
__device__ __forceinline__ bf16x8 gen_beta_eta(const float* lb, const float* eta, int r, int q, int lane) {
  // loads unconditional (every index in range), the triangle applied by selects: no branches
  const int gq = lane >> 4;
  const float lbr = MOM ? lb[r] : 0.f;
  bf16x8 f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int u = 32 * q + 8 * gq + e;
    const float et = eta[u];
    float v;
    if (MOM) {
      const float x = -et * __builtin_amdgcn_exp2f(lb[u] - lbr);
      v = u >= r ? x : 0.f;
    } else {
      v = u == r ? -et : 0.f;
    }
    f[e] = static_cast<bf16>(v);
  }
  return f;
}
// A'[t][u] = A(u -> t - 1) = exp2(LA[t-1] - LA[u]) for u <= t - 1 (t, u chunk-local).
__device__ __forceinline__ bf16x8 gen_decay_to(const float* la, int t, int q, int lane) {
  const int gq = lane >> 4;
  const float lat = la[t > 0 ? t - 1 : 0];
  bf16x8 f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int u = 32 * q + 8 * gq + e;
    const float x = __builtin_amdgcn_exp2f(lat - la[u]);
    f[e] = static_cast<bf16>(u <= t - 1 ? x : 0.f);
  }
  return f;
}
// Window weights Wg[s][r] = w(r, r - s) for 0 <= r - s < e, chained k order over the targets r
// (slot e < 4: r = 32 q + 4 gq + e; e >= 4: r = 32 q + 16 + 4 gq + e - 4); s = row - HT.
__device__ __forceinline__ bf16x8 gen_wgate(const Geom& g, const float* wl, const float* ug, int t0, int srow, int q,
                                            int lane) {
  const int gq = lane >> 4;
  const int s = srow - HT;
  bf16x8 f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int r = 32 * q + (e < 4 ? 4 * gq + e : 16 + 4 * gq + e - 4);
    const int j = r - s;
    float v = 0.f;
    if (j >= 0 && j < g.e) v = win_w(g, wl, t0, ug, t0 - HT, t0 + r, j);
    f[e] = static_cast<bf16>(v);
  }
  return f;
}

}  // namespace cp
}  // namespace atlas
