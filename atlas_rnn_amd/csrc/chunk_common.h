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
}  // namespace cp
}  // namespace atlas
