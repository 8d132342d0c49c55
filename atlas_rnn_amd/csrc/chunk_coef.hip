// chunk_coef.hip - the forward walks' chunk records on the matrix cores (bf16 inputs, 64-token
// chunks, window <= 17), for plans whose backward forms its own coefficients (chunk_bwd.hip).
//
// One wave per (chunk, row), four independent waves per workgroup, no workgroup barrier: every
// chunk is in flight at once (C3: 2048 waves, 8 per CU) and its latency chain (loads, scans, two
// small products, stores) overlaps with the others'. The record and the Ws block are the ones the
// per-source chains of coef.hip produce (same layout, no mid point):
//   acoef[t] = a_{t-1} = At[t], kcoef[t] = kappa_{t-1} = -Kt[t] (the coefficients of S_c, Z_c in
//   S_{t-1}), endc = (a, kappa, b, 0) of the whole chunk, wsend[s] = Ws[s, end] = -cs_s,
//   wzend[s] = Wz[s, end] = cz_s, and wsh[t][s] = Ws[s, t-1] = -Wy[s][t],
// where Wy = Bd C' (Bd[s][r] the window band: the weight of source s in the window of target r)
// and C' = BE DA^T (C'[r][t]: the coefficient of g_r in S_{t-1}) from the prefix arrays of the
// chunk's decay / lr / beta: two 64-wide products per chunk instead of one serial 64-step chain per
// source. Sources s = 0 .. 63 + H are the tokens t0 - H + s (H = e - 1); the rest of the 96 source
// slots are zero.
//
// Operands (v_mfma_f32_16x16x32_bf16; lane l: gq = l >> 4, m = l & 15):
//   C' tile (rb, tb) = sum_q BE(rb, q) DA(tb, q), k = u = 32 q + 8 gq + e (natural order), the
//     operands generated in registers: one product of separable factors per entry (exp2(LA[t-1])
//     exp2(-LA[u]), eta_u exp2(LB[u]) exp2(-LB[r]), formed once per token) where the chunk's
//     summed log2 decays stay above -120, else exp2 of the differences (<= 0); tiles rb > tb
//     and the k-steps outside u in [16 rb, 16 tb + 14] are zero and skipped;
//   Wy tile (sb, tb) = sum_q Band(sb, q) C'(q, tb), k = r in the chained order of the accumulator
//     tiles (slots e < 4: r = 32 q + 4 gq + e; e >= 4: r = 32 q + 16 + 4 gq + e - 4), so the C'
//     accumulators are the B operand as they stand (pack_frag); the band slots are read from the
//     wave's gate table. Band(sb, q) is zero unless 16 sb - 16 <= 32 q + 31 and 32 q <= 16 sb + 15.
#include <type_traits>

#include "chunk_common.h"

namespace atlas {

namespace cpf {
using namespace cp;

constexpr int NT = 256;
constexpr int NWV = NT / 64;         // chunks per workgroup (one per wave)
constexpr int SPM = CL + kHaloPad;   // source slots of the record and of the Ws rows (96)
constexpr int REC = CoefRec<CL>::SIZE;
constexpr int R_KCOEF = CL, R_ENDC = 2 * CL, R_WSEND = R_ENDC + 4, R_WZEND = R_WSEND + SPM, R_WSMID = R_WZEND + SPM;
static_assert(R_WSMID + 2 * SPM + 4 == REC && R_WSMID % 4 == 0, "record layout");

// per wave: the prefix arrays, the end coefficients of the targets and the window band
struct WvSm {
  alignas(16) float la[CL], lb[CL], eta[CL], gs[CL], gz[CL];
  // separable factors (chunks whose total log2 decays stay above -kSepRange): A(u -> t - 1) =
  // qa[t] pa[u], -eta_u B(r -> u) = pb[u] qb[r]
  alignas(16) float qa[CL], pa[CL], pb[CL], qb[CL];
  // Bd[s][r] = w(r, j), s = r + H - j: the weight of source s in the window of target r (zero
  // outside the window and past T)
  alignas(16) BandRows Bd;
};

// Makes the wave's LDS writes visible to its own later reads (no workgroup barrier).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// BE(rb, q): rows r = 16 rb + m, k = u natural: -eta_u B(r -> u) = -eta_u exp2(LB[u] - LB[r]) for
// u >= r (momentum; MASK false: every u of the fragment is >= every r); -eta_r at u = r without.
template <bool MOM, bool MASK>
__device__ __forceinline__ bf16x8 gen_be(const WvSm& ws, int r, int q, int gq) {
  const int u0 = 32 * q + 8 * gq;
  const float4 e0 = *reinterpret_cast<const float4*>(&ws.eta[u0]), e1 = *reinterpret_cast<const float4*>(&ws.eta[u0 + 4]);
  const float etu[8] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
  bf16x8 f;
  if constexpr (MOM) {
    const float4 b0 = *reinterpret_cast<const float4*>(&ws.lb[u0]), b1 = *reinterpret_cast<const float4*>(&ws.lb[u0 + 4]);
    const float lbu[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    const float lbr = ws.lb[r];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = -etu[e] * __builtin_amdgcn_exp2f(lbu[e] - lbr);
      f[e] = static_cast<bf16>(!MASK || u0 + e >= r ? x : 0.f);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = static_cast<bf16>(u0 + e == r ? -etu[e] : 0.f);
  }
  return f;
}
// The same fragments from the separable factors (one product per entry instead of an exp2).
template <bool MOM, bool MASK>
__device__ __forceinline__ bf16x8 gen_be_sep(const WvSm& ws, int r, int q, int gq) {
  const int u0 = 32 * q + 8 * gq;
  bf16x8 f;
  if constexpr (MOM) {
    const float4 b0 = *reinterpret_cast<const float4*>(&ws.pb[u0]), b1 = *reinterpret_cast<const float4*>(&ws.pb[u0 + 4]);
    const float pbu[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    const float qbr = ws.qb[r];
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = static_cast<bf16>(!MASK || u0 + e >= r ? pbu[e] * qbr : 0.f);
  } else {
    f = gen_be<false, MASK>(ws, r, q, gq);
  }
  return f;
}
template <bool MASK>
__device__ __forceinline__ bf16x8 gen_da_sep(const WvSm& ws, int t, int q, int gq) {
  const int u0 = 32 * q + 8 * gq;
  const float4 a0 = *reinterpret_cast<const float4*>(&ws.pa[u0]), a1 = *reinterpret_cast<const float4*>(&ws.pa[u0 + 4]);
  const float pau[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
  const float qat = ws.qa[t];
  bf16x8 f;
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = static_cast<bf16>(!MASK || u0 + e <= t - 1 ? qat * pau[e] : 0.f);
  return f;
}
// DA(tb, q) as the B operand: lane supplies DA[t = 16 tb + m][u = 32 q + 8 gq + e] = A(u -> t - 1)
// (u <= t - 1; MASK false: the whole fragment lies below the diagonal)
template <bool MASK>
__device__ __forceinline__ bf16x8 gen_da(const WvSm& ws, int t, int q, int gq) {
  const int u0 = 32 * q + 8 * gq;
  const float4 a0 = *reinterpret_cast<const float4*>(&ws.la[u0]), a1 = *reinterpret_cast<const float4*>(&ws.la[u0 + 4]);
  const float lau[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
  const float lat = ws.la[t > 0 ? t - 1 : 0];
  bf16x8 f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float x = __builtin_amdgcn_exp2f(lat - lau[e]);
    f[e] = static_cast<bf16>(!MASK || u0 + e <= t - 1 ? x : 0.f);
  }
  return f;
}
// Band(sb, q): lane supplies Bd[s = 16 sb + m][r] for the chained slots r = 32 q + 4 gq + 0..3 and
// 32 q + 16 + 4 gq + 0..3 (two 8-byte reads)
__device__ __forceinline__ bf16x8 gen_band(const WvSm& ws, int s, int q, int gq) {
  const uint2 a = *reinterpret_cast<const uint2*>(&ws.Bd[s][32 * q + 4 * gq]);
  const uint2 b = *reinterpret_cast<const uint2*>(&ws.Bd[s][32 * q + 16 + 4 * gq]);
  return __builtin_bit_cast(bf16x8, u32x4v{a.x, a.y, b.x, b.y});
}

// The window weights of target token tc (lane = target): lag gates w[j] = gate[tc][j], or token
// gates w[j] = gate[tc - j] (clamped at token 0; masked by the caller). NJ >= e loads, all issued
// before any use; lags past e repeat the last one.
template <int NJ>
__device__ __forceinline__ void gates_ld(const Geom& g, const bf16* __restrict__ gate, size_t rowbase, int tc,
                                         bf16 (&gx)[EMAX]) {
  if (g.gate_mode == GATE_LAG) {
    const bf16* p = gate + (rowbase + tc) * g.e;
#pragma unroll
    for (int j = 0; j < NJ; ++j) gx[j] = p[min(j, g.e - 1)];
  } else {
#pragma unroll
    for (int j = 0; j < NJ; ++j) gx[j] = gate[rowbase + max(tc - j, 0)];
  }
}

// cs_s, cz_s = sum_r Bd[s][r] (cgS[r], cgZ[r]) over the targets r = s - H + j (j < e) whose window
// holds source s; NJ >= e terms, branch-free (clamped reads, masked weights).
template <int NJ>
__device__ __forceinline__ void end_sources(const WvSm& ws, int s, int H, int e, float& cs, float& cz) {
  const int sc = min(s, SRC - 1);
  bf16 wv[NJ];
  float gv[NJ], zv[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {   // every read first (none predicated), then the sums
    const int rc = min(max(s - H + j, 0), CL - 1);
    wv[j] = ws.Bd[sc][rc];
    gv[j] = ws.gs[rc];
    zv[j] = ws.gz[rc];
  }
  cs = 0.f;
  cz = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int r = s - H + j;
    const float wgt = static_cast<float>(wv[j]) * (j < e && r >= 0 && r < CL && s < SRC ? 1.f : 0.f);
    cs += wgt * gv[j];
    cz += wgt * zv[j];
  }
}

constexpr bool c_tile(int rb, int tb) { return rb <= tb; }                    // C'(rb, tb) nonzero
constexpr bool c_step(int rb, int tb, int q) { return 32 * q <= 16 * tb + 14 && 32 * q + 31 >= 16 * rb; }
constexpr bool band_step(int sb, int q) { return 16 * sb - HT <= 32 * q + 31 && 32 * q <= 16 * sb + 15; }

template <bool MOM>
__global__ __launch_bounds__(NT) void k_chunk_coef_fwd(const Geom g, const bf16* __restrict__ decay,
                                                       const bf16* __restrict__ lr, const bf16* __restrict__ beta,
                                                       const bf16* __restrict__ gate, float* __restrict__ rec_all,
                                                       bf16* __restrict__ wsh_all) {
  if (geom_skip(g)) return;
  __shared__ WvSm wsm[NWV];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int c = blockIdx.x * NWV + wv, bh = blockIdx.y;
  if (c >= g.nc) return;   // wave-uniform; no workgroup barrier follows
  WvSm& ws = wsm[wv];
  const int gq = lane >> 4, m = lane & 15;
  const int t0 = c * CL, H = g.H, e = g.e;
  const size_t rowbase = (size_t)bh * g.T;
  const bool real = t0 + lane < g.T;

  // ---- inputs (lane = target r): the scalars (the identity past T) and the window weights; every
  // load unconditional (clamped index) and issued before the first use
  const int tc = t0 + min(lane, g.T - 1 - t0);
  const bf16 xa = decay[rowbase + tc], xe = lr[rowbase + tc], xb = MOM ? beta[rowbase + tc] : static_cast<bf16>(0.f);
  bf16 gx[EMAX];
#pragma unroll
  for (int j = 0; j < EMAX; ++j) gx[j] = static_cast<bf16>(1.f);
  if (g.gate_mode != GATE_NONE) {
    if (e <= 4) gates_ld<4>(g, gate, rowbase, tc, gx);
    else if (e <= 8) gates_ld<8>(g, gate, rowbase, tc, gx);
    else gates_ld<EMAX>(g, gate, rowbase, tc, gx);
  }
  const float al = real ? static_cast<float>(xa) : 1.f, et = real ? static_cast<float>(xe) : 0.f;
  const float be = real ? static_cast<float>(xb) : 1.f;

  // ---- prefix arrays (LA, LB, eta), the coefficients of S_c, Z_c in S_{t-1}, the end coefficients
  const float lav = wave_prefix_sum(fmaxf(__log2f(al), kLogFloor), lane);
  const float lbv = wave_prefix_sum(fmaxf(__log2f(be), kLogFloor), lane);
  ws.la[lane] = lav;
  ws.lb[lane] = lbv;
  ws.eta[lane] = et;
  // separable factors (chunk_common.h): the prefix sums only decrease, so lane 63 holds the lowest
  const bool sep = __shfl(lav, 63, 64) >= -kSepRange && (!MOM || __shfl(lbv, 63, 64) >= -kSepRange);
  if (sep) {   // wave-uniform
    const float lap = __shfl(lav, lane > 0 ? lane - 1 : 0, 64);
    ws.qa[lane] = lane > 0 ? __builtin_amdgcn_exp2f(lap) : 1.f;
    ws.pa[lane] = __builtin_amdgcn_exp2f(-lav);
    if (MOM) {
      ws.pb[lane] = -et * __builtin_amdgcn_exp2f(lbv);
      ws.qb[lane] = __builtin_amdgcn_exp2f(-lbv);
    }
  }
  for (int i = lane; i < (int)(sizeof(BandRows) / 16); i += 64)
    reinterpret_cast<u32x4v*>(&ws.Bd[0][0])[i] = u32x4v{0u, 0u, 0u, 0u};
  wave_sync();
#pragma unroll
  for (int j = 0; j < EMAX; ++j)   // zero past T and (token gates) for sources before token 0
    if (j < e)
      ws.Bd[lane + H - j][lane] =
          real && (g.gate_mode != GATE_TOKEN || t0 + lane - j >= 0) ? gx[j] : static_cast<bf16>(0.f);
  Tri ex = tri_prev_lane(wave_scan<true>(Tri{al, -et * be, be}, lane));
  if (lane == 0) ex = tri_id();
  float* rec = rec_all + ((size_t)bh * g.nc + c) * REC;
  rec[lane] = ex.a;
  rec[R_KCOEF + lane] = -ex.k;
  {   // the chunk read backwards: lane j holds target r = 63 - j
    const float ar = __shfl(al, 63 - lane, 64), er = __shfl(et, 63 - lane, 64), br = __shfl(be, 63 - lane, 64);
    const Tri inc = wave_scan<false>(Tri{ar, -er * br, br}, lane);
    Tri ey = tri_prev_lane(inc);
    if (lane == 0) ey = tri_id();
    const int r = 63 - lane;
    const bool rr = t0 + r < g.T;
    ws.gs[r] = rr ? ey.k - er * ey.a : 0.f;
    ws.gz[r] = rr ? ey.b : 0.f;
    if (lane == 63) *reinterpret_cast<float4*>(rec + R_ENDC) = make_float4(inc.a, -inc.k, inc.b, 0.f);
  }
  if (lane < 2 * SPM / 4 + 1)   // wsmid, wzmid, midc
    *reinterpret_cast<float4*>(rec + R_WSMID + 4 * lane) = make_float4(0.f, 0.f, 0.f, 0.f);
  wave_sync();

  // ---- cs, cz of sources s = lane and 64 + lane
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int s = lane + 64 * h;
    float cs, cz;
    if (e <= 4) end_sources<4>(ws, s, H, e, cs, cz);
    else if (e <= 8) end_sources<8>(ws, s, H, e, cs, cz);
    else end_sources<EMAX>(ws, s, H, e, cs, cz);
    if (s < SPM) {
      rec[R_WSEND + s] = -cs;
      rec[R_WZEND + s] = cz;
    }
  }

  // ---- C' = BE DA^T (tiles rb <= tb); the operands from the separable factors where they exist
  f32x4 cpt[4][4];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) cpt[rb][tb] = zero4();
  auto cprime = [&](auto sepc) {
    constexpr bool SEP = decltype(sepc)::value;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      bf16x8 fda[4];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        if (!c_step(0, tb, q)) continue;
        const int t = 16 * tb + m;
        if (32 * q + 32 > 16 * tb) fda[tb] = SEP ? gen_da_sep<true>(ws, t, q, gq) : gen_da<true>(ws, t, q, gq);
        else fda[tb] = SEP ? gen_da_sep<false>(ws, t, q, gq) : gen_da<false>(ws, t, q, gq);
      }
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        if (!c_step(rb, 3, q)) continue;
        const int r = 16 * rb + m;
        bf16x8 fbe;
        if (32 * q < 16 * rb + 15) fbe = SEP ? gen_be_sep<MOM, true>(ws, r, q, gq) : gen_be<MOM, true>(ws, r, q, gq);
        else fbe = SEP ? gen_be_sep<MOM, false>(ws, r, q, gq) : gen_be<MOM, false>(ws, r, q, gq);
#pragma unroll
        for (int tb = rb; tb < 4; ++tb)
          if (c_step(rb, tb, q)) cpt[rb][tb] = mma_bf16(fbe, fda[tb], cpt[rb][tb]);
      }
    }
  };
  if (sep) cprime(std::true_type{});
  else cprime(std::false_type{});

  // ---- Wy = Band C', stored as wsh[t][s] = -Wy[s][t] (lane: sources 16 sb + 4 gq + i of target
  // 16 tb + m; 8-byte stores; 0 - x keeps the empty slots +0). Only the source tiles sb <= tb + 1
  // are stored: Ws[s, t - 1] is zero past s = t + H - 1 (H <= 16), and the walks read no more.
  const rsrc_t rw = make_rsrc(wsh_all + ((size_t)bh * g.nc + c) * CL * SPM, (uint32_t)(CL * SPM * sizeof(bf16)));
  bf16x8 fband[5][2];
#pragma unroll
  for (int sb = 0; sb < 5; ++sb)
#pragma unroll
    for (int q = 0; q < 2; ++q)
      if (band_step(sb, q)) fband[sb][q] = gen_band(ws, 16 * sb + m, q, gq);
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    bf16x8 fc[2];
#pragma unroll
    for (int q = 0; q < 2; ++q)
      if (c_tile(2 * q, tb)) fc[q] = pack_frag(cpt[2 * q][tb], cpt[2 * q + 1][tb]);
    const uint32_t row = (uint32_t)(((16 * tb + m) * SPM + 4 * gq) * sizeof(bf16));
#pragma unroll
    for (int sb = 0; sb < 6; ++sb) {
      if (sb > tb + 1) continue;   // Ws[s, t - 1] = 0 for s > t + H - 1: never stored, never read
      f32x4 acc = zero4();
#pragma unroll
      for (int q = 0; q < 2; ++q)
        if (sb < 5 && band_step(sb, q) && c_tile(2 * q, tb)) acc = mma_bf16(fband[sb < 5 ? sb : 0][q], fc[q], acc);
      bst8(rw, row + 32 * sb, u32x2v{pack_bf16x2(0.f - acc[0], 0.f - acc[1]), pack_bf16x2(0.f - acc[2], 0.f - acc[3])});
    }
  }
}

}  // namespace cpf

bool chunk_coef_fwd_supported(const Geom& g) {
  return g.Lc == cp::CL && g.H <= cp::HT && g.e <= cp::EMAX && g.Lmid == 0 && g.H == g.e - 1;
}

// The forward records (coef, [BH][nc] records of CoefRec<64>::SIZE floats) and Ws blocks (wsh,
// [BH][nc][64][96] bf16) of every 64-token chunk.
hipError_t launch_chunk_coef_fwd(const Geom& g, const bf16* decay, const bf16* lr, const bf16* beta, const bf16* gate,
                                 float* coef, bf16* wsh, hipStream_t stream) {
  if (!chunk_coef_fwd_supported(g) || (g.momentum && !beta) || (g.gate_mode != GATE_NONE && !gate))
    return hipErrorInvalidValue;
  prof_name(KID_FWD_COEF, "k_chunk_coef_fwd");
  prof_begin(KID_FWD_COEF, stream);
  const dim3 grid((g.nc + cpf::NWV - 1) / cpf::NWV, g.BH);
  if (g.momentum)
    hipLaunchKernelGGL((cpf::k_chunk_coef_fwd<true>), grid, dim3(cpf::NT), 0, stream, g, decay, lr, beta, gate, coef, wsh);
  else
    hipLaunchKernelGGL((cpf::k_chunk_coef_fwd<false>), grid, dim3(cpf::NT), 0, stream, g, decay, lr, beta, gate, coef, wsh);
  prof_end(KID_FWD_COEF, stream);
  return hipGetLastError();
}

}  // namespace atlas
