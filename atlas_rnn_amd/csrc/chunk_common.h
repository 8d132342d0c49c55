// chunk_common.h - pieces of the backward walk with in-kernel coefficients (chunk_bwd.hip; bf16
// inputs, d_k = d_v = 64, window <= 17, no scan_chunk_len clamp, no carried buffer).
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
constexpr float kLogFloor = -100.f;
// A chunk whose prefix sums LA, LB end above -kSepRange has separable decay factors: exp2(LA[t] -
// LA[u]) = exp2(LA[t]) exp2(-LA[u]) with both factors fp32 normal numbers (within 2^(+-120)).
constexpr float kSepRange = 120.f;

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

// Operand generators (row = lane & 15 of the tile, k slots natural: k = 32 q + 8 gq + e; lane passed in).
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

constexpr int PB = 72;     // LDS pitch (bf16 elements) of 64-wide rows (16-byte aligned rows)
constexpr int EMAX = 17;   // longest window
// chunk coefficient record (floats): cs, cz (sources: coefficients of G_s in S, Z at the chunk end),
// cgS, cgZ (targets: of g_r in S, Z at the chunk end), the chunk transition (a, k, b, 0)
constexpr int R_CS = 0, R_CZ = SRC, R_GS = 2 * SRC, R_GZ = 2 * SRC + CL, R_TR = 2 * SRC + 2 * CL;
constexpr int REC = R_TR + 4;   // 292

// Per chunk: the end record and the prefix arrays (LA, LB, eta, beta; the coefficients At, Kt of
// (S_c, Z_c) in S_{t-1} and B1 of Z_c in Z_{t-1}).
struct ChunkCoef {
  alignas(16) float co[REC];
  alignas(16) float la[CL], lb[CL], eta[CL], At[CL], Kt[CL], B1[CL], be[CL];
};
// the window band of a chunk: Bd[s][r] = w(r, r + HT - s) for 0 <= r + HT - s < e (zero elsewhere),
// the weight of source s in the window of target r (w: the lag gate, the token gate of the source,
// or 1; zero for targets past T)
typedef bf16 BandRows[SRC][PB];
typedef bf16 Rows64[CL][PB];

// window weight of lag j for chunk target r (from the staged band)
__device__ __forceinline__ float cw(const BandRows& Bd, int r, int j) { return static_cast<float>(Bd[r + HT - j][r]); }

// One wave (lane = target r, its scalars al, et, be; the identity past T): the chunk's end
// coefficients cgS, cgZ of every target and the chunk transition.
__device__ __forceinline__ void chunk_end_scan(int T, float al0, float et0, float be0, int t0, int lane,
                                               ChunkCoef& kc) {
  // lane j holds target r = 63 - j (the chunk read backwards)
  const float al = __shfl(al0, 63 - lane, 64), et = __shfl(et0, 63 - lane, 64), be = __shfl(be0, 63 - lane, 64);
  const Tri x{al, -et * be, be};
  const Tri inc = wave_scan<false>(x, lane);
  Tri ex = tri_prev_lane(inc);
  if (lane == 0) ex = tri_id();
  const int r = 63 - lane;
  const bool real = t0 + r < T;
  kc.co[R_GS + r] = real ? ex.k - et * ex.a : 0.f;
  kc.co[R_GZ + r] = real ? ex.b : 0.f;
  if (lane == 63) { kc.co[R_TR] = inc.a; kc.co[R_TR + 1] = inc.k; kc.co[R_TR + 2] = inc.b; kc.co[R_TR + 3] = 0.f; }
}
// cs_s, cz_s over NJ >= e lags, branch-free: every read issued first (clamped, none predicated),
// then the masked sums.
template <int NJ>
__device__ __forceinline__ void end_sources_nj(const BandRows& Bd, const ChunkCoef& kc, int s, int e, float& cs,
                                               float& cz) {
  bf16 wv[NJ];
  float gv[NJ], zv[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int rc = min(max(s - HT + j, 0), CL - 1);
    wv[j] = Bd[s][rc];
    gv[j] = kc.co[R_GS + rc];
    zv[j] = kc.co[R_GZ + rc];
  }
  cs = 0.f;
  cz = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int r = s - HT + j;
    const float wgt = static_cast<float>(wv[j]) * (j < e && r >= 0 && r < CL ? 1.f : 0.f);
    cs += wgt * gv[j];
    cz += wgt * zv[j];
  }
}
// Thread s < 80: the per-source end coefficients from cgS / cgZ (after chunk_end_scan and the band):
// cs_s = sum_j w(s - HT + j, j) cgS[s - HT + j], cz_s likewise with cgZ (Bd[s][r] = w(r, j)).
__device__ __forceinline__ void chunk_end_sources(const Geom& g, const BandRows& Bd, ChunkCoef& kc, int s) {
  if (s >= 0 && s < SRC) {
    float cs, cz;
    if (g.e <= 4) end_sources_nj<4>(Bd, kc, s, g.e, cs, cz);
    else if (g.e <= 8) end_sources_nj<8>(Bd, kc, s, g.e, cs, cz);
    else end_sources_nj<EMAX>(Bd, kc, s, g.e, cs, cz);
    kc.co[R_CS + s] = cs;
    kc.co[R_CZ + s] = cz;
  }
}
// The two factors of C' = BE DA^T (C'[r][t]: the coefficient of g_r in S_{t-1}) from the prefix
// arrays: DA[t][u] = A(u -> t - 1) (u < t), BE[r][u] = -eta_u B(r -> u) (u >= r; without momentum
// -eta_r at u = r). Item i < 512: row i >> 3, columns 8 (i & 7) .. +7; loads unconditional, the
// triangles applied by selects.
template <bool MOM>
__device__ __forceinline__ void gen_tables(const ChunkCoef& kc, Rows64& DA, Rows64& BE, int i) {
  const int row = i >> 3, u0 = (i & 7) * 8;
  const float4 a0 = *reinterpret_cast<const float4*>(&kc.la[u0]), a1 = *reinterpret_cast<const float4*>(&kc.la[u0 + 4]);
  const float lau[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
  const float lat = kc.la[row > 0 ? row - 1 : 0];
  const float4 e0 = *reinterpret_cast<const float4*>(&kc.eta[u0]), e1 = *reinterpret_cast<const float4*>(&kc.eta[u0 + 4]);
  const float etu[8] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
  const float4 b0 = *reinterpret_cast<const float4*>(&kc.lb[u0]), b1 = *reinterpret_cast<const float4*>(&kc.lb[u0 + 4]);
  const float lbu[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
  const float lbr = kc.lb[row];
  bf16x8 da, be;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int u = u0 + e;
    const float x = __builtin_amdgcn_exp2f(lat - lau[e]);
    da[e] = static_cast<bf16>(u <= row - 1 ? x : 0.f);
    float v;
    if (MOM) {
      const float y = -etu[e] * __builtin_amdgcn_exp2f(lbu[e] - lbr);
      v = u >= row ? y : 0.f;
    } else {
      v = u == row ? -etu[e] : 0.f;
    }
    be[e] = static_cast<bf16>(v);
  }
  *reinterpret_cast<bf16x8*>(&DA[row][u0]) = da;
  *reinterpret_cast<bf16x8*>(&BE[row][u0]) = be;
}
// One wave (lane = target, its scalars): the chunk's prefix arrays LA, LB (log2 prefix sums, floored),
// eta, beta, and At, Kt, B1.
__device__ __forceinline__ void chunk_prefix(float al, float et, float be, int lane, ChunkCoef& kc) {
  kc.la[lane] = wave_prefix_sum(fmaxf(__log2f(al), kLogFloor), lane);
  kc.lb[lane] = wave_prefix_sum(fmaxf(__log2f(be), kLogFloor), lane);
  kc.eta[lane] = et;
  kc.be[lane] = be;
  const Tri inc = wave_scan<true>(Tri{al, -et * be, be}, lane);
  Tri ex = tri_prev_lane(inc);
  if (lane == 0) ex = tri_id();
  kc.At[lane] = ex.a;
  kc.Kt[lane] = ex.k;
  kc.B1[lane] = ex.b;
}

}  // namespace cp
}  // namespace atlas
