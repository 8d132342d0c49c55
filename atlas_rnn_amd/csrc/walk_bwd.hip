// walk_bwd.hip - specialised reverse walk of the backward pass for bf16 inputs with d_k = d_v = 64.
//
// Replaces k_bwd_seg (seg_bwd.hip) for the configurations the specialised forward walks cover; the
// adjoint aggregates, the segment scan, the scalar gradients (k_bwd_scalar), the fixup and the
// dS_ref reduction are shared with the general path and see the same per-chunk records.
// Chunks of 32 tokens, sources s = 0 .. 47 (the e - 1 <= 16 halo tokens, then the chunk),
// processed last to first within a segment in three phases, software-pipelined so that phase C of
// chunk c+1 and phase A of chunk c share one barrier interval (two barriers per chunk):
//   phase A  bf16 copies of the chunk-end adjoint for the matrix cores; delta = S_ref phi - v
//            (-> LDS), K = psi phi^T (kept) and Q = Ws o K (-> LDS), the state term S_in^T dy of
//            dpsi (kept), the Grams <dS_end, S_in> ..., and the chunk-start adjoint (the
//            transposed chunk transition, in the owners' fp32 registers)
//   phase B  P = dy delta^T, Q' = Ws o P (-> LDS) and Lm = K o P (scalar-gradient record);
//            dDelta = Wz_end dZ_end phi - Ws_end dS_end phi - Q^T dy (-> LDS, dv) with hS, hZ
//   phase C  dpsi (dq), dphi (dk), dS_ref += dDelta^T phi, the scalar records
// The inputs of chunk c-1 are staged (double buffered by chunk parity) during phase B of chunk c;
// delta, the adjoint copies and the phase-A reductions are double buffered by chunk parity too.
// The chunk-start states come from the forward walk in the fragment layout of walk_common.h and
// feed the matrix cores without going through LDS.
#include "mem_common.h"
#include "mem_params.h"
#include "seg_common.h"
#include "seg_fixup.h"
#include "walk_common.h"

namespace atlas {

namespace wb {

constexpr int D = 64;
constexpr int CH = 32;          // backward chunk length
constexpr int SP = 48;          // source rows with data: halo (<= 16) + chunk
constexpr int NST = SP / 16;    // 3 source tiles
constexpr int SPR = 64;         // LDS rows of source-indexed matrices (rows SP.. stay zero: k = 32 steps)
constexpr int PD = D + 16;      // pitch of 64-wide bf16 rows
constexpr int SPM = CH + kHaloPad;   // 64: pitch of the per-source arrays in HBM (records, Ws, Lm)
constexpr int WP = SPR + 8;     // 72: LDS pitch of the Ws rows [tau][s] (columns SP.. stay zero)
constexpr int QP = CH + 8;      // 40: LDS pitch of Q^T / Q'^T rows [s][tau]
constexpr int REC = CoefRec<CH>::SIZE;   // 328
constexpr int R_ACOEF = 0, R_KCOEF = CH, R_ENDC = 2 * CH, R_WSEND = 2 * CH + 4, R_WZEND = R_WSEND + SPM;
constexpr int REC4 = REC / 4;   // 82
constexpr int HMAX = 16;
typedef ScalarBlock<CH> SB;
static_assert(SB::SPM == SPM, "scalar record pitch");
static_assert(R_WSEND % 4 == 0 && R_WZEND % 4 == 0 && REC % 4 == 0, "record alignment");

struct Stage {
  alignas(16) bf16 phi[SPR][PD];
  alignas(16) bf16 psi[CH][PD];
  alignas(16) bf16 dy[CH][PD];
  alignas(16) bf16 wsh[CH][WP];
  alignas(16) float rec[REC];
};

struct Smem {
  Stage st[2];                        // staged inputs, by chunk parity
  alignas(16) bf16 dl[2][SPR][PD];    // delta[s][i], by chunk parity
  alignas(16) bf16 dD[SPR][PD];       // dDelta[s][i]
  alignas(16) bf16 QT[SPR][QP];       // Q^T[s][tau]
  alignas(16) bf16 QpT[SPR][QP];      // Q'^T[s][tau]
  alignas(16) bf16 dSeT[2][D][PD];    // chunk-end adjoint, transposed (dSeT[k][i] = dS_end[i][k]), by parity
  alignas(16) bf16 dZeT[2][D][PD];
  alignas(16) float carry[2][HMAX][2 * D];   // halo partials (dv | dphi) handed to the previous chunk
  // scalar-gradient sums, one slot per contributing wave (summed in a fixed order when the chunk's
  // record is written, so the result does not depend on the order the waves finish in)
  float hS[4][SPM], hZ[4][SPM];       // [it1][s]
  float fS[2][4][CH], fZ[2][4][CH];   // [chunk parity][kt][tau]
  float red[2][kSegWaves][4];         // Gram partials, by chunk parity
};
static_assert(sizeof(Smem) <= 160 * 1024, "one workgroup per CU: at most 160 KB of LDS");

// Register prefetch: the staged inputs (loaded one chunk ahead of their staging) and the operands
// consumed from registers in phase A (v of the wave's delta tiles, the saved chunk-start states).
struct StagePf {
  u32x4v phi, x;        // phi row vector (tid < 384); psi (waves 0-3) or dy (waves 4-7) row vector
  u32x4v wsh, rec;
};
struct RegPf {
  u32x2v v[2];
  u32x4v sin[2], zin[2];   // chunk-start S, Z fragments (kt, q = 0, 1)
};

}  // namespace wb

template <bool MAPE, int HC, bool BUF>
__global__ __launch_bounds__(kSegThreads) void k_walk_bwd(const Geom g, const BwdPtrs<bf16> a, const SegGeom sg,
                                                            const BwdSegPtrs p) {
  using namespace wb;
  if (geom_skip(g)) return;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  Smem& sm = *reinterpret_cast<Smem*>(smem_raw);
  const int tid = threadIdx.x, lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform (scalar) wave index
  const int gq = lane >> 4, m = lane & 15;
  const int seg = blockIdx.x, bh = blockIdx.y;
  const int H = HC >= 0 ? HC : g.H;
  const int c_begin = seg * sg.G, c_end = min(g.nc, c_begin + sg.G);
  const size_t DD = (size_t)D * D;
  const size_t sbase = (size_t)bh * DD;
  const int seg_tail0 = min(g.T, c_end * CH) - H;
  // roles (every wave does the same work; source tile 3, s = 48 .. 63, is zero padding)
  const int qw = w & 1, kt = w >> 1;     // owned adjoint tiles: rows 32 qw + 16 u, columns 16 kt
  const int it1 = w & 3;                 // delta / dDelta tiles: rows 16 it1, sources 16 st1(u)
  const int s1a = w >> 2;                // st1(u) = s1a + 2 u
  const int tt = w & 1, stm = w >> 1;    // K / P tile: targets 16 tt, sources 16 stm
  // dpsi tile: features 16 kt, targets 16 qw; dphi tiles: features 16 kt, sources 16 (qw + 2 u)

  const uint32_t row_bytes = (uint32_t)g.T * (D * 2);
  const rsrc_t rk = make_rsrc(a.k + (size_t)bh * g.T * D, row_bytes);
  const rsrc_t rv = make_rsrc(a.v + (size_t)bh * g.T * D, row_bytes);
  const rsrc_t rq = make_rsrc(a.q + (size_t)bh * g.T * D, row_bytes);
  const rsrc_t rdy = make_rsrc(a.dy ? a.dy + (size_t)bh * g.T * D : a.q, a.dy ? row_bytes : 0u);
  const rsrc_t rrec = make_rsrc(p.coef + (size_t)bh * g.nc * REC, (uint32_t)g.nc * (REC * 4));
  const rsrc_t rwsh = make_rsrc(reinterpret_cast<const bf16*>(p.wsh) + (size_t)bh * g.nc * CH * SPM,
                                (uint32_t)g.nc * (CH * SPM * 2));
  const rsrc_t rdq = make_rsrc(a.dq + (size_t)bh * g.T * D, row_bytes);
  const rsrc_t rdk = make_rsrc(a.dk + (size_t)bh * g.T * D, row_bytes);
  const rsrc_t rdv = make_rsrc(a.dv + (size_t)bh * g.T * D, row_bytes);
  const unsigned char* states = reinterpret_cast<const unsigned char*>(p.rw) + (size_t)bh * g.ncb * kStateBlk;

  // per-thread staging offsets (relative to token t0 / chunk c)
  const int sv_s = tid >> 3, sv_c8 = tid & 7;
  const uint32_t o_phi = (tid < SP * 8 && sv_s < H + CH) ? (uint32_t)((sv_s - H) * (D * 2) + sv_c8 * 16) : kOob;
  const int l_phi = tid < SP * 8 ? sv_s * PD + sv_c8 * 8 : -1;
  const int xr = (tid & 255) >> 3;
  const uint32_t o_x = (uint32_t)(xr * (D * 2) + sv_c8 * 16);
  const int l_x = xr * PD + sv_c8 * 8;
  const uint32_t o_wsh = tid < CH * (SP / 8) ? (uint32_t)((tid / (SP / 8)) * (SPM * 2) + (tid % (SP / 8)) * 16) : kOob;
  const int l_wsh = tid < CH * (SP / 8) ? (tid / (SP / 8)) * WP + (tid % (SP / 8)) * 8 : -1;
  const uint32_t o_rec = tid < REC4 ? (uint32_t)(tid * 16) : kOob;
  uint32_t o_v[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int s = 16 * (s1a + 2 * u) + m;
    o_v[u] = s < H + CH ? (uint32_t)((s - H) * (D * 2) + (16 * it1 + 4 * gq) * 2) : kOob;
  }

  auto sp_load = [&](StagePf& pf, int c) {
    const uint32_t tb = (uint32_t)(c * CH) * (D * 2);
    pf.phi = bld16(rk, o_phi + tb);
    pf.x = bld16(w < 4 ? rq : rdy, o_x + tb);   // waves 0-3: psi rows, 4-7: dy rows
    pf.wsh = bld16(rwsh, o_wsh + (uint32_t)c * (CH * SPM * 2));
    pf.rec = bld16(rrec, o_rec + (uint32_t)c * (REC * 4));
  };
  auto sp_store = [&](const StagePf& pf, Stage& st) {
    if (l_phi >= 0) {
      u32x4v x = pf.phi;
      if constexpr (MAPE) x = map_bf16x8(x, g.map_deg);
      *reinterpret_cast<u32x4v*>(&st.phi[0][0] + l_phi) = x;
    }
    if (tid < 256) {
      u32x4v x = pf.x;
      if constexpr (MAPE) x = map_bf16x8(x, g.map_deg);
      *reinterpret_cast<u32x4v*>(&st.psi[0][0] + l_x) = x;
    } else {
      *reinterpret_cast<u32x4v*>(&st.dy[0][0] + l_x) = pf.x;
    }
    if (l_wsh >= 0) *reinterpret_cast<u32x4v*>(&st.wsh[0][0] + l_wsh) = pf.wsh;
    if (tid < REC4) *reinterpret_cast<u32x4v*>(&st.rec[tid * 4]) = pf.rec;
  };
  auto rp_load = [&](RegPf& pf, int c) {
    const uint32_t tb = (uint32_t)(c * CH) * (D * 2);
#pragma unroll
    for (int u = 0; u < 2; ++u) pf.v[u] = bld8(rv, o_v[u] + tb);
    const unsigned char* blk = states + (size_t)c * kStateBlk;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      pf.sin[q] = *reinterpret_cast<const u32x4v*>(blk + frag_off(kt, q, lane));
      pf.zin[q] = *reinterpret_cast<const u32x4v*>(blk + kStateBytes + frag_off(kt, q, lane));
    }
  };

  // ---- constants: S_ref rows 16 it1 (A operand of delta) and S_ref^T columns 16 kt (A of S_ref^T dDelta)
  bf16x8 sref_f[2], srefT_f[2];
  {
    const float* sr = a.S_ref + sbase;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const float* r0 = sr + (size_t)(16 * it1 + m) * D + 32 * q + 8 * gq;
      const float4 x0 = *reinterpret_cast<const float4*>(r0);
      const float4 x1 = *reinterpret_cast<const float4*>(r0 + 4);
      bf16x8 f;
      f[0] = static_cast<bf16>(x0.x); f[1] = static_cast<bf16>(x0.y); f[2] = static_cast<bf16>(x0.z);
      f[3] = static_cast<bf16>(x0.w); f[4] = static_cast<bf16>(x1.x); f[5] = static_cast<bf16>(x1.y);
      f[6] = static_cast<bf16>(x1.z); f[7] = static_cast<bf16>(x1.w);
      sref_f[q] = f;
      bf16x8 ft;
#pragma unroll
      for (int e = 0; e < 8; ++e) ft[e] = static_cast<bf16>(sr[(size_t)(32 * q + 8 * gq + e) * D + 16 * kt + m]);
      srefT_f[q] = ft;
    }
  }

  // ---- adjoint at the segment end (owned tiles u: rows 32 qw + 16 u + 4 gq + r, column 16 kt + m)
  float dS[2][4], dZ[2][4], dsr[2][4];
  {
    const float* sa = p.seg_adj + ((size_t)bh * sg.nseg + seg) * 2 * DD;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const size_t off = (size_t)(32 * qw + 16 * u + 4 * gq + r) * D + 16 * kt + m;
        dS[u][r] = sa[off];
        dZ[u][r] = sa[DD + off];
        dsr[u][r] = 0.f;
      }
  }

  // ---- zero the padding rows, the carries and the accumulators
  for (int idx = tid; idx < (SPR - SP) * PD; idx += kSegThreads) {
    const int rr = SP + idx / PD, cc = idx % PD;
    sm.st[0].phi[rr][cc] = bf16(0.f);
    sm.st[1].phi[rr][cc] = bf16(0.f);
    sm.dl[0][rr][cc] = bf16(0.f);
    sm.dl[1][rr][cc] = bf16(0.f);
    sm.dD[rr][cc] = bf16(0.f);
  }
  for (int idx = tid; idx < (SPR - SP) * QP; idx += kSegThreads) {
    const int rr = SP + idx / QP, cc = idx % QP;
    sm.QT[rr][cc] = bf16(0.f);
    sm.QpT[rr][cc] = bf16(0.f);
  }
  for (int idx = tid; idx < CH * (WP - SP); idx += kSegThreads) {
    const int rr = idx / (WP - SP), cc = SP + idx % (WP - SP);
    sm.st[0].wsh[rr][cc] = bf16(0.f);
    sm.st[1].wsh[rr][cc] = bf16(0.f);
  }
  for (int idx = tid; idx < 2 * HMAX * 2 * D; idx += kSegThreads) (&sm.carry[0][0][0])[idx] = 0.f;
  for (int idx = tid; idx < 4 * SPM; idx += kSegThreads) { (&sm.hS[0][0])[idx] = 0.f; (&sm.hZ[0][0])[idx] = 0.f; }
  for (int idx = tid; idx < 8 * CH; idx += kSegThreads) { (&sm.fS[0][0][0])[idx] = 0.f; (&sm.fZ[0][0][0])[idx] = 0.f; }

  // Per-chunk context: token range, halo routing.
  struct Ctx {
    int c, t0, t1, L, tail0;
    bool first;
    float* cur_carry;
    const float* prev_carry;
  };
  auto ctx = [&](int c) {
    Ctx x;
    x.c = c;
    x.t0 = c * CH;
    x.t1 = min(g.T, x.t0 + CH);
    x.L = x.t1 - x.t0;
    x.tail0 = x.t1 - H;
    x.first = c == c_begin;
    x.cur_carry = &sm.carry[c & 1][0][0];
    x.prev_carry = &sm.carry[(c + 1) & 1][0][0];
    return x;
  };
  // Routes the (dv | dphi) values of source s, features f0 .. f0+3 (half 0: dv, 1: dphi): halo
  // sources to the previous chunk's carry (or the segment's halo record), the chunk's last e-1
  // tokens plus the next chunk's carry, the segment's last e-1 tokens to the tail record.
  auto route = [&](const Ctx& x, int s, int f0, int half, float* val, const rsrc_t& dst, const u32x2v& raw) {
    const int pp = x.t0 - H + s;
    if (s >= H + x.L || pp < 0) return;
    if (s < H) {
      float* o = x.first ? p.halo_part + (((size_t)bh * sg.nseg + seg) * H + s) * (2 * D) : x.cur_carry + s * (2 * D);
      *reinterpret_cast<float4*>(o + half * D + f0) = make_float4(val[0], val[1], val[2], val[3]);
      return;
    }
    if (pp >= x.tail0) {
      const float4 cv = *reinterpret_cast<const float4*>(x.prev_carry + (pp - x.tail0) * (2 * D) + half * D + f0);
      val[0] += cv.x; val[1] += cv.y; val[2] += cv.z; val[3] += cv.w;
    }
    if (pp >= seg_tail0) {
      float* o = p.tail_part + (((size_t)bh * sg.nseg + seg) * H + (pp - seg_tail0)) * (2 * D) + half * D + f0;
      *reinterpret_cast<float4*>(o) = make_float4(val[0], val[1], val[2], val[3]);
      return;
    }
    if constexpr (MAPE) {
      if (half == 1) {
        val[0] *= poly_map_grad(__builtin_bit_cast(float, raw[0] << 16), g.map_deg);
        val[1] *= poly_map_grad(__builtin_bit_cast(float, raw[0] & 0xffff0000u), g.map_deg);
        val[2] *= poly_map_grad(__builtin_bit_cast(float, raw[1] << 16), g.map_deg);
        val[3] *= poly_map_grad(__builtin_bit_cast(float, raw[1] & 0xffff0000u), g.map_deg);
      }
    }
    u32x2v o;
    o[0] = pack_bf16x2(val[0], val[1]);
    o[1] = pack_bf16x2(val[2], val[3]);
    bst8(dst, (uint32_t)((pp * D + f0) * 2), o);
  };

  // values handed from phase A of a chunk to its phases B and C
  f32x4 kmat = zero4(), TS = zero4(), TZ = zero4();
  float wt[4] = {0.f, 0.f, 0.f, 0.f};
  u32x2v mq = {0u, 0u}, mk[2] = {{0u, 0u}, {0u, 0u}};
  StagePf sp;
  RegPf rp;

  // ================================ phase A ================================
  // delta tiles C[i][s], K tile C[tau][s] (Q = Ws o K), the state term of dpsi C[k][tau] =
  // sum_i S_in[i][k] dy[tau][i], the chunk transition terms, the Grams; operands first, then the
  // matrix products, then the epilogues and LDS stores. Ends by loading the registers of chunk c-1.
  auto phaseA = [&](int c) {
    const int ln = launder(lane) & 63;
    const int gq = ln >> 4, m = ln & 15;
    const Stage& st = sm.st[c & 1];
    const float* rec = st.rec;
    const int t0 = c * CH;
    if constexpr (MAPE) {   // raw q, k of this lane's dq / dk elements for the map derivative
      mq = bld8(rq, (uint32_t)((t0 + 16 * qw + m) * (D * 2) + (16 * kt + 4 * gq) * 2));
#pragma unroll
      for (int u = 0; u < 2; ++u)
        mk[u] = bld8(rk, (uint32_t)((t0 - H + 16 * (qw + 2 * u) + m) * (D * 2) + (16 * kt + 4 * gq) * 2));
    }
    f32x4 dl_acc[2], xa[2], xk[2];
    {
      bf16x8 fphi[2][2], fpk[2], fps[2], fdy[2];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int q = 0; q < 2; ++q) fphi[u][q] = frag_row_l(&st.phi[0][0], PD, 16 * (s1a + 2 * u), 32 * q, ln);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        fpk[q] = frag_row_l(&st.phi[0][0], PD, 16 * stm, 32 * q, ln);
        fps[q] = frag_row_l(&st.psi[0][0], PD, 16 * tt, 32 * q, ln);
        const int tau = 16 * qw + m;
        const uint2 lo = *reinterpret_cast<const uint2*>(&st.dy[tau][32 * q + 4 * gq]);
        const uint2 hi = *reinterpret_cast<const uint2*>(&st.dy[tau][32 * q + 16 + 4 * gq]);
        const u32x4v bv = {lo.x, lo.y, hi.x, hi.y};
        fdy[q] = __builtin_bit_cast(bf16x8, bv);
      }
      const bf16x8 fpsiT = frag_tr_l(&st.psi[0][0], PD, 16 * kt, 0, ln);
      bf16x8 fya[2], fyk[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        fya[u] = frag_tr_scaled_l(&st.dy[0][0], PD, 32 * qw + 16 * u, 0, rec + R_ACOEF, ln);
        fyk[u] = frag_tr_scaled_l(&st.dy[0][0], PD, 32 * qw + 16 * u, 0, rec + R_KCOEF, ln);
      }
      const s16x4 wv = tr4_l(&st.wsh[0][0], WP, 16 * tt, 16 * stm, ln);
#pragma unroll
      for (int r = 0; r < 4; ++r) wt[r] = bf16_bits_to_f32((unsigned short)wv[r]);

#pragma unroll
      for (int u = 0; u < 2; ++u) {
        dl_acc[u] = mma_bf16(sref_f[0], fphi[u][0], zero4());
        dl_acc[u] = mma_bf16(sref_f[1], fphi[u][1], dl_acc[u]);
      }
      kmat = mma_bf16(fps[0], fpk[0], zero4());
      kmat = mma_bf16(fps[1], fpk[1], kmat);
      TS = mma_bf16(__builtin_bit_cast(bf16x8, rp.sin[0]), fdy[0], zero4());
      TZ = mma_bf16(__builtin_bit_cast(bf16x8, rp.zin[0]), fdy[0], zero4());
      TS = mma_bf16(__builtin_bit_cast(bf16x8, rp.sin[1]), fdy[1], TS);
      TZ = mma_bf16(__builtin_bit_cast(bf16x8, rp.zin[1]), fdy[1], TZ);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        xa[u] = mma_bf16(fya[u], fpsiT, zero4());
        xk[u] = mma_bf16(fyk[u], fpsiT, zero4());
      }
    }
    {   // delta = acc - v -> LDS; Q -> LDS
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const u32x2v vv = rp.v[u];
        store4<bf16>(&sm.dl[c & 1][16 * (s1a + 2 * u) + m][16 * it1 + 4 * gq],
                     dl_acc[u][0] - __builtin_bit_cast(float, vv[0] << 16),
                     dl_acc[u][1] - __builtin_bit_cast(float, vv[0] & 0xffff0000u),
                     dl_acc[u][2] - __builtin_bit_cast(float, vv[1] << 16),
                     dl_acc[u][3] - __builtin_bit_cast(float, vv[1] & 0xffff0000u));
      }
      store4<bf16>(&sm.QT[16 * stm + m][16 * tt + 4 * gq], wt[0] * kmat[0], wt[1] * kmat[1], wt[2] * kmat[2],
                   wt[3] * kmat[3]);
    }
    {   // fS, fZ (partial over this wave's 16 features, summed over the rows)
      const int tau = 16 * qw + m;
      const float4 ps = lds_bf16x4(&st.psi[tau][16 * kt + 4 * gq]);
      const float fs = xsum_rows(TS[0] * ps.x + TS[1] * ps.y + TS[2] * ps.z + TS[3] * ps.w);
      const float fz = xsum_rows(TZ[0] * ps.x + TZ[1] * ps.y + TZ[2] * ps.z + TZ[3] * ps.w);
      if (gq == 0) { sm.fS[c & 1][kt][tau] = fs; sm.fZ[c & 1][kt][tau] = fz; }
    }
    {   // Grams <dS_end, S_in>, <dS_end, Z_in>, <dZ_end, Z_in> (fragment (kt, qw) holds the owned elements;
        // selects, not a runtime index, so that the prefetch registers stay registers)
      const bf16x8 fs = __builtin_bit_cast(bf16x8, qw ? rp.sin[1] : rp.sin[0]);
      const bf16x8 fz = __builtin_bit_cast(bf16x8, qw ? rp.zin[1] : rp.zin[0]);
      float gss = 0.f, gsz = 0.f, gzz = 0.f;
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float sv = static_cast<float>(fs[4 * u + r]), zv = static_cast<float>(fz[4 * u + r]);
          gss += dS[u][r] * sv; gsz += dS[u][r] * zv; gzz += dZ[u][r] * zv;
        }
      gss = xsum_rows(row_sum16(gss)); gsz = xsum_rows(row_sum16(gsz)); gzz = xsum_rows(row_sum16(gzz));
      if (ln == 0) { sm.red[c & 1][w][0] = gss; sm.red[c & 1][w][1] = gsz; sm.red[c & 1][w][2] = gzz; }
    }
    {   // the chunk-end adjoint's bf16 copies (read by phases B, C), then the chunk-start adjoint:
        //   dS_in = a dS_end + sum_t a_{t-1} dy_t psi_t^T,  dZ_in = b dZ_end - kappa dS_end - sum_t kappa_{t-1} dy_t psi_t^T
      const float ae = rec[R_ENDC], ke = rec[R_ENDC + 1], be = rec[R_ENDC + 2];
      if (BUF && c == 0) {   // chunk 0's end adjoint, for the carried buffer's terms (bufwalk.hip)
        float* ba = p.buf_adj + (size_t)bh * bufw::kAdjFloats;
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int off = (32 * qw + 16 * u + 4 * gq + r) * D + 16 * kt + m;
            ba[off] = dS[u][r];
            ba[DD + off] = dZ[u][r];
          }
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int i0 = 32 * qw + 16 * u + 4 * gq;
        store4<bf16>(&sm.dSeT[c & 1][16 * kt + m][i0], dS[u][0], dS[u][1], dS[u][2], dS[u][3]);
        store4<bf16>(&sm.dZeT[c & 1][16 * kt + m][i0], dZ[u][0], dZ[u][1], dZ[u][2], dZ[u][3]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float lam = ae * dS[u][r] + xa[u][r];
          const float mu = g.momentum ? (be * dZ[u][r] - ke * dS[u][r] - xk[u][r]) : 0.f;
          dS[u][r] = lam;
          dZ[u][r] = mu;
        }
      }
      if (c == 0) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const size_t off = sbase + (size_t)(32 * qw + 16 * u + 4 * gq + r) * D + 16 * kt + m;
            a.dS0[off] = dS[u][r];
            if (g.momentum && a.dZ0) a.dZ0[off] = dZ[u][r];
          }
      }
    }
    // this chunk's register operands are consumed: load the previous chunk's
    if (c - 1 >= c_begin) rp_load(rp, c - 1);
  };

  // ================================ phase B ================================
  // P tile C[tau][s] = dy delta^T (Lm = K o P, Q' = Ws o P); dDelta tiles C[i][s] =
  // Wz_end dZ_end phi - Ws_end dS_end phi - sum_tau dy Q (hS, hZ, dv)
  auto phaseB = [&](int c) {
    const int ln = launder(lane) & 63;
    const int gq = ln >> 4, m = ln & 15;
    const Stage& st = sm.st[c & 1];
    const float* rec = st.rec;
    const Ctx x = ctx(c);
    float* blk = p.scal + ((size_t)bh * g.nc + c) * SB::SIZE;
    bf16x8 fy[2], fd[2], fp[2][2], fsT[2], fzT[2], fq[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      fy[q] = frag_row_l(&st.dy[0][0], PD, 16 * tt, 32 * q, ln);
      fd[q] = frag_row_l(&sm.dl[c & 1][0][0], PD, 16 * stm, 32 * q, ln);
      fsT[q] = frag_tr_l(&sm.dSeT[c & 1][0][0], PD, 16 * it1, 32 * q, ln);
      fzT[q] = frag_tr_l(&sm.dZeT[c & 1][0][0], PD, 16 * it1, 32 * q, ln);
#pragma unroll
      for (int u = 0; u < 2; ++u) fp[u][q] = frag_row_l(&st.phi[0][0], PD, 16 * (s1a + 2 * u), 32 * q, ln);
    }
    const bf16x8 fyT = frag_tr_l(&st.dy[0][0], PD, 16 * it1, 0, ln);
#pragma unroll
    for (int u = 0; u < 2; ++u) fq[u] = frag_row_l(&sm.QT[0][0], QP, 16 * (s1a + 2 * u), 0, ln);
    float4 dlv[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) dlv[u] = lds_bf16x4(&sm.dl[c & 1][16 * (s1a + 2 * u) + m][16 * it1 + 4 * gq]);

    f32x4 pm = mma_bf16(fy[0], fd[0], zero4());
    pm = mma_bf16(fy[1], fd[1], pm);
    f32x4 as[2], az[2], aq[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      as[u] = mma_bf16(fsT[0], fp[u][0], zero4());
      az[u] = mma_bf16(fzT[0], fp[u][0], zero4());
      aq[u] = mma_bf16(fyT, fq[u], zero4());
      as[u] = mma_bf16(fsT[1], fp[u][1], as[u]);
      az[u] = mma_bf16(fzT[1], fp[u][1], az[u]);
    }

    {
      float* lp = blk + (unsigned)(SB::LM + (16 * tt + 4 * gq) * SPM + 16 * stm + m);
#pragma unroll
      for (int r = 0; r < 4; ++r) lp[r * SPM] = kmat[r] * pm[r];
    }
    store4<bf16>(&sm.QpT[16 * stm + m][16 * tt + 4 * gq], wt[0] * pm[0], wt[1] * pm[1], wt[2] * pm[2], wt[3] * pm[3]);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int s = 16 * (s1a + 2 * u) + m, i0 = 16 * it1 + 4 * gq;
      const float wz = rec[R_WZEND + s], ws = rec[R_WSEND + s];
      const float dlr[4] = {dlv[u].x, dlv[u].y, dlv[u].z, dlv[u].w};
      float dd[4], hs = 0.f, hz = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        dd[r] = wz * az[u][r] - ws * as[u][r] - aq[u][r];
        hs += dlr[r] * as[u][r];
        hz += dlr[r] * az[u][r];
      }
      hs = xsum_rows(hs);
      hz = xsum_rows(hz);
      if (gq == 0) { sm.hS[it1][s] = hs; sm.hZ[it1][s] = hz; }
      store4<bf16>(&sm.dD[s][i0], dd[0], dd[1], dd[2], dd[3]);
      float val[4] = {-dd[0], -dd[1], -dd[2], -dd[3]};
      route(x, s, i0, 0, val, rdv, u32x2v{0u, 0u});
    }
  };

  // ================================ phase C ================================
  // dpsi tile C[k][tau] = a_{tau-1} S_in^T dy - kappa_{tau-1} Z_in^T dy - sum_s phi_s Q'[tau][s];
  // dphi tiles C[k][s] = Wz_end dZ_end^T delta - Ws_end dS_end^T delta - sum_tau psi Q' + S_ref^T dDelta;
  // dS_ref += dDelta^T phi on the owned tiles; the chunk's scalar-gradient record
  auto phaseC = [&](int c) {
    const int ln = launder(lane) & 63;
    const int gq = ln >> 4, m = ln & 15;
    const Stage& st = sm.st[c & 1];
    const float* rec = st.rec;
    const Ctx x = ctx(c);
    bf16x8 fphT[2], fqpT[2], fdl[2][2], fzE[2], fsE[2], fdd[2][2], fqp[2], fddT[2][2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      fphT[q] = frag_tr_l(&st.phi[0][0], PD, 16 * kt, 32 * q, ln);
      fqpT[q] = frag_tr_l(&sm.QpT[0][0], QP, 16 * qw, 32 * q, ln);
      fzE[q] = frag_row_l(&sm.dZeT[c & 1][0][0], PD, 16 * kt, 32 * q, ln);
      fsE[q] = frag_row_l(&sm.dSeT[c & 1][0][0], PD, 16 * kt, 32 * q, ln);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        fdl[u][q] = frag_row_l(&sm.dl[c & 1][0][0], PD, 16 * (qw + 2 * u), 32 * q, ln);
        fdd[u][q] = frag_row_l(&sm.dD[0][0], PD, 16 * (qw + 2 * u), 32 * q, ln);
        fddT[u][q] = frag_tr_l(&sm.dD[0][0], PD, 32 * qw + 16 * u, 32 * q, ln);
      }
    }
    const bf16x8 fpsT = frag_tr_l(&st.psi[0][0], PD, 16 * kt, 0, ln);
#pragma unroll
    for (int u = 0; u < 2; ++u) fqp[u] = frag_row_l(&sm.QpT[0][0], QP, 16 * (qw + 2 * u), 0, ln);

    f32x4 a7 = mma_bf16(fphT[0], fqpT[0], zero4());
    a7 = mma_bf16(fphT[1], fqpT[1], a7);
    f32x4 a1[2], a2[2], a3[2], a4[2], a6[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      a1[u] = mma_bf16(fzE[0], fdl[u][0], zero4());
      a2[u] = mma_bf16(fsE[0], fdl[u][0], zero4());
      a4[u] = mma_bf16(srefT_f[0], fdd[u][0], zero4());
      a6[u] = mma_bf16(fddT[u][0], fphT[0], zero4());
      a3[u] = mma_bf16(fpsT, fqp[u], zero4());
      a1[u] = mma_bf16(fzE[1], fdl[u][1], a1[u]);
      a2[u] = mma_bf16(fsE[1], fdl[u][1], a2[u]);
      a4[u] = mma_bf16(srefT_f[1], fdd[u][1], a4[u]);
      a6[u] = mma_bf16(fddT[u][1], fphT[1], a6[u]);
    }

    {   // dq
      const int tau = 16 * qw + m;
      const float ac = rec[R_ACOEF + tau], kc = rec[R_KCOEF + tau];
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = ac * TS[r] - kc * TZ[r] - a7[r];
      if constexpr (MAPE) {
        v[0] *= poly_map_grad(__builtin_bit_cast(float, mq[0] << 16), g.map_deg);
        v[1] *= poly_map_grad(__builtin_bit_cast(float, mq[0] & 0xffff0000u), g.map_deg);
        v[2] *= poly_map_grad(__builtin_bit_cast(float, mq[1] << 16), g.map_deg);
        v[3] *= poly_map_grad(__builtin_bit_cast(float, mq[1] & 0xffff0000u), g.map_deg);
      }
      u32x2v o;
      o[0] = pack_bf16x2(v[0], v[1]);
      o[1] = pack_bf16x2(v[2], v[3]);
      bst8(rdq, (uint32_t)(((x.t0 + tau) * D + 16 * kt + 4 * gq) * 2), o);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {   // dk
      const int s = 16 * (qw + 2 * u) + m;
      const float wz = rec[R_WZEND + s], ws = rec[R_WSEND + s];
      float val[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) val[r] = wz * a1[u][r] - ws * a2[u][r] - a3[u][r] + a4[u][r];
      route(x, s, 16 * kt + 4 * gq, 1, val, rdk, mk[u]);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) dsr[u][r] += a6[u][r];

    // scalar-gradient record of the chunk (hS, hZ after phase B; fS, fZ, Grams after phase A)
    float* blk = p.scal + ((size_t)bh * g.nc + c) * SB::SIZE;
    if (tid >= 256 && tid < 256 + SPM) {
      const int s = tid - 256;
      blk[SB::HS + s] = (sm.hS[0][s] + sm.hS[1][s]) + (sm.hS[2][s] + sm.hS[3][s]);
      blk[SB::HZ + s] = (sm.hZ[0][s] + sm.hZ[1][s]) + (sm.hZ[2][s] + sm.hZ[3][s]);
    } else if (tid >= 384 && tid < 384 + CH) {
      const int t = tid - 384;
      const float(&fs)[4][CH] = sm.fS[c & 1];
      const float(&fz)[4][CH] = sm.fZ[c & 1];
      blk[SB::FS + t] = (fs[0][t] + fs[1][t]) + (fs[2][t] + fs[3][t]);
      blk[SB::FZ + t] = (fz[0][t] + fz[1][t]) + (fz[2][t] + fz[3][t]);
    } else if (tid >= 448 && tid < 452) {
      const int j = tid - 448;
      float sum = 0.f;
      if (j < 3) {
#pragma unroll
        for (int ww = 0; ww < kSegWaves; ++ww) sum += sm.red[c & 1][ww][j];
      }
      blk[SB::GRAM + j] = sum;
    }
  };

  // ---- software pipeline over the chunks (last to first), two barriers per chunk:
  //   [phase C of chunk c+1 | phase A of chunk c] -> [phase B of chunk c | staging of chunk c-1]
  sp_load(sp, c_end - 1);
  sp_store(sp, sm.st[(c_end - 1) & 1]);
  if (c_end - 2 >= c_begin) sp_load(sp, c_end - 2);
  rp_load(rp, c_end - 1);
  __syncthreads();
  phaseA(c_end - 1);
  __syncthreads();
  phaseB(c_end - 1);
  if (c_end - 2 >= c_begin) {
    sp_store(sp, sm.st[(c_end - 2) & 1]);
    if (c_end - 3 >= c_begin) sp_load(sp, c_end - 3);
  }
  __syncthreads();
  for (int c = c_end - 2; c >= c_begin; --c) {
    phaseC(c + 1);
    phaseA(c);
    __syncthreads();
    phaseB(c);
    if (c - 1 >= c_begin) {
      sp_store(sp, sm.st[(c - 1) & 1]);
      if (c - 2 >= c_begin) sp_load(sp, c - 2);
    }
    __syncthreads();
  }
  phaseC(c_begin);

  // ---- segment output: dS_ref partial
  float* dst = p.dsref_part + ((size_t)bh * sg.nseg + seg) * DD;
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int r = 0; r < 4; ++r) dst[(size_t)(32 * qw + 16 * u + 4 * gq + r) * D + 16 * kt + m] = dsr[u][r];
}

size_t walk_bwd_smem_bytes() { return sizeof(wb::Smem); }

template <bool MAPE, int HC, bool BUF = false>
hipError_t launch_walk_bwd_h(const Geom& g, const BwdPtrs<bf16>& a, const SegGeom& sg, const BwdSegPtrs& p,
                             hipStream_t stream) {
  const size_t smem = sizeof(wb::Smem);
  const hipError_t err = set_dyn_smem(reinterpret_cast<const void*>(&k_walk_bwd<MAPE, HC, BUF>), smem);
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL((k_walk_bwd<MAPE, HC, BUF>), dim3(sg.nseg, g.BH), dim3(kSegThreads), smem, stream, g, a, sg, p);
  return hipGetLastError();
}
template <bool MAPE>
hipError_t launch_walk_bwd_m(const Geom& g, const BwdPtrs<bf16>& a, const SegGeom& sg, const BwdSegPtrs& p,
                             hipStream_t stream) {
  // a carried buffer (window > 1): the generic-halo kernel that also leaves chunk 0's end adjoint
  if (p.buf_adj) return launch_walk_bwd_h<MAPE, -1, true>(g, a, sg, p, stream);
  switch (g.H) {
    case 0: return launch_walk_bwd_h<MAPE, 0>(g, a, sg, p, stream);
    case 3: return launch_walk_bwd_h<MAPE, 3>(g, a, sg, p, stream);
    case 7: return launch_walk_bwd_h<MAPE, 7>(g, a, sg, p, stream);
    default: return launch_walk_bwd_h<MAPE, -1>(g, a, sg, p, stream);
  }
}
hipError_t launch_walk_bwd_kernel(const Geom& g, const BwdPtrs<bf16>& a, const SegGeom& sg, const BwdSegPtrs& p,
                                  hipStream_t stream) {
  return g.map_mode == MAP_ELEMENTWISE ? launch_walk_bwd_m<true>(g, a, sg, p, stream)
                                       : launch_walk_bwd_m<false>(g, a, sg, p, stream);
}

// ---------------------------------------------------------------------------------------------
// Scalar gradients of the specialised path, one wave per 32-token chunk (four chunks per
// workgroup), as the reverse-mode form of the chunk's coefficient recurrences. Lane s < 48 owns
// source s and lane 48 the chunk prefix; every lane runs the same branch-free code:
//   forward   Wz_t = beta_t Wz_{t-1} + w(s, t),   Ws_t = alpha_t Ws_{t-1} + eta_t Wz_t,   a_t = alpha_t a_{t-1}
//   reverse   gWs_t = G_t + alpha_{t+1} gWs_{t+1},  gWz_t = Hz_t + eta_t gWs_t + beta_{t+1} gWz_{t+1},
//             ga_t = Ga_t + alpha_{t+1} ga_{t+1}
// A source starts from Wz = Ws = 0 with the window weights as input and the direct terms
// G_t = -Lm[t+1][s] (t < 31), G_31 = -hS[s], Hz_31 = hZ[s], Ga = 0 from the walk's record. The
// prefix lane starts from Wz = 1 (so that Wz_t = b_t and Ws_t = kappa_t) with no input, and
// G_t = -fZ[t+1], G_31 = -<dS_end, Z_in>, Hz_31 = <dZ_end, Z_in>, Ga_t = fS[t+1], Ga_31 = <dS_end, S_in>.
// Per step a lane contributes
//   dalpha_t += gWs_t Ws_{t-1} + ga_t a_{t-1},  deta_t += gWs_t Wz_t,  dbeta_t += gWz_t Wz_{t-1},
// and a source's window-weight gradient is dw(s, t) = gWz_t. The contributions are summed over
// lane quads with DPP, then over the quads through LDS. The step scalars are the same for every
// lane and are broadcast from lane t with v_readlane; all arithmetic is fp32.
// ---------------------------------------------------------------------------------------------
namespace wb {
constexpr int kChainWaves = 4;
constexpr int kWalkWindow = SP - CH + 1;   // 17: the largest window of the specialised path
constexpr int NSRC = SP;          // 48 source lanes; lane NSRC runs the prefix chain
constexpr int RP = CH + 1;        // pitch of the window-weight rows
constexpr int NQD = 13;           // lane quads holding live lanes (0 .. 51)
constexpr int QDP = 16;           // pitch of the per-step quad rows
struct ChainSmem {   // static LDS: kChainWaves * 6.3 KB
  union {
    float W[NSRC][RP];                  // window weights w(s, t) of the sources
    struct {
      alignas(16) float red[3][CH][QDP];   // quad sums of the alpha / eta / beta contributions of step t
      float dw[CH * kWalkWindow + 1];      // window-weight gradients [t][j]; the last slot takes masked writes
    } r;
  } u[kChainWaves];
};
__device__ __forceinline__ float quad_sum(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0xB1, 0xf, 0xf, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x4E, 0xf, 0xf, false));
  return x;
}
}  // namespace wb

// Workgroups x >= nchain run the segment fixup of segment x - nchain instead (seg_fixup.h): both
// read only what the reverse walk wrote, so one launch carries both.
static_assert(64 * wb::kChainWaves == kThreads, "the fixup workgroups share the launch's block size");
__global__ __launch_bounds__(64 * wb::kChainWaves) void k_scalar_chain(const Geom g, const BwdPtrs<bf16> a,
                                                                         const BwdSegPtrs p, const SegGeom sg,
                                                                         int nchain) {
  using namespace wb;
  if (geom_skip(g)) return;
  if ((int)blockIdx.x >= nchain) {   // workgroup-uniform
    bwd_seg_fixup<bf16, D, false>(g, a, sg, p, 1, blockIdx.x - nchain, blockIdx.y);
    return;
  }
  __shared__ ChainSmem smc;
  const int lane = lane_id();
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = blockIdx.x * kChainWaves + wv, bh = blockIdx.y;
  if (c >= g.nc) return;   // wave-uniform: no barriers below
  const int H = g.H, e = g.e;
  const int t0 = c * CH, L = min(g.T, t0 + CH) - t0;
  const size_t tb = (size_t)bh * g.T;
  const float* blk = p.scal + ((size_t)bh * g.nc + c) * SB::SIZE;
  auto& U = smc.u[wv];
  const bool src = lane < NSRC, pre = lane == NSRC;

  // step scalars in lane t (padded steps: alpha = beta = 1, eta = 0; beta = 0 without momentum)
  float al = 1.f, et = 0.f, be = 1.f;
  if (lane < L) {
    al = to_f32(a.decay[tb + t0 + lane]);
    et = to_f32(a.lr[tb + t0 + lane]);
    be = g.momentum ? to_f32(a.beta[tb + t0 + lane]) : 0.f;
  }
  // direct terms of this lane. Every lane issues the same loads (no load sits in a lane-dependent
  // branch, so they are all in flight together); the prefix lane's terms come from lane broadcasts
  // in the reverse loop.
  const int col = src ? lane : 0;
  float lmv[CH - 1];
#pragma unroll
  for (int t = 0; t < CH - 1; ++t) lmv[t] = blk[SB::LM + (t + 1) * SPM + col];
  const float fsl = blk[SB::FS + (lane & (CH - 1))], fzl = blk[SB::FZ + (lane & (CH - 1))];
  const float gram = blk[SB::GRAM + (lane & 3)];
  const float hs = blk[SB::HS + col], hz = blk[SB::HZ + col];

  // window weights of the sources: W[s][t] = w(s, t) for j = t + H - s in [0, e)
  for (int idx = lane; idx < NSRC * RP; idx += 64) (&U.W[0][0])[idx] = 0.f;
  __builtin_amdgcn_wave_barrier();
  for (int idx = lane; idx < CH * e; idx += 64) {
    const int t = idx / e, j = idx % e, s = t + H - j;
    float wgt = 0.f;
    if (t < L) {
      if (g.gate_mode == GATE_LAG) wgt = to_f32(a.gate[(tb + t0 + t) * e + j]);
      else if (g.gate_mode == GATE_TOKEN)   // a buffer source carries its gate inside B: weight 1
        wgt = t0 + t - j >= 0 ? to_f32(a.gate[tb + t0 + t - j]) : (g.has_buf ? 1.f : 0.f);
      else wgt = 1.f;
    }
    if (s >= 0 && s < NSRC) U.W[s][t] = wgt;
  }
  __builtin_amdgcn_wave_barrier();
  float wrow[CH];
  {
    const int row = src ? lane : 0;
#pragma unroll
    for (int t = 0; t < CH; ++t) wrow[t] = src ? U.W[row][t] : 0.f;
  }
  __builtin_amdgcn_wave_barrier();

  // forward
  float wsp[CH], wzc[CH], wzp[CH];
  {
    float wz = pre ? 1.f : 0.f, ws = 0.f;
#pragma unroll
    for (int t = 0; t < CH; ++t) {
      const float A = lane_bcast(al, t), E = lane_bcast(et, t), B = lane_bcast(be, t);
      wzp[t] = wz;
      wsp[t] = ws;
      wz = B * wz + wrow[t];
      ws = A * ws + E * wz;
      wzc[t] = wz;
    }
  }
  // a_{t-1} = prod_{tau < t} alpha_tau in lane t (an exclusive product scan over the lanes; it is the
  // same for every source, so it is broadcast per step instead of held in 32 registers per lane)
  float apl = al;
#pragma unroll
  for (int d = 1; d < CH; d <<= 1) {
    const float y = __shfl_up(apl, d, 64);
    if (lane >= d) apl *= y;
  }
  {
    const float sh = __shfl_up(apl, 1, 64);
    apl = lane == 0 ? 1.f : sh;
  }
  // reverse (branch-free: masked stores go to a dummy slot). The step scalars are broadcast again
  // from laundered copies, so that the forward loop's broadcasts are not held in scalar registers
  // across both loops; the direct terms G_t, Ga_t are formed per step.
  {
    const float alr = launder_f(al), ber = launder_f(be), etr = launder_f(et);
    const float gss = lane_bcast(gram, 0), gsz = lane_bcast(gram, 1), gzz = lane_bcast(gram, 2);
    const float hz_end = src ? hz : (pre ? gzz : 0.f);
    const bool live = lane <= NSRC;
    const bool quad_head = (lane & 3) == 0 && lane < 4 * NQD;
    const int qrow = quad_head ? (lane >> 2) : QDP - 1;   // column QDP - 1 is never read
    float gws = 0.f, gwz = 0.f, ga = 0.f;
#pragma unroll
    for (int t = CH - 1; t >= 0; --t) {
      const float A1 = t + 1 < CH ? lane_bcast(alr, t + 1) : 0.f;
      const float B1 = t + 1 < CH ? lane_bcast(ber, t + 1) : 0.f;
      const float E = lane_bcast(etr, t);
      float dG, dA;
      if (t < CH - 1) {   // compile-time branch; the broadcasts stay outside lane-dependent selects
        const float fs = lane_bcast(fsl, t + 1), fz = lane_bcast(fzl, t + 1);
        dG = src ? -lmv[t] : (pre ? -fz : 0.f);
        dA = pre ? fs : 0.f;
      } else {
        dG = src ? -hs : (pre ? -gsz : 0.f);
        dA = pre ? gss : 0.f;
      }
      gws = dG + A1 * gws;
      gwz = (t == CH - 1 ? hz_end : 0.f) + E * gws + B1 * gwz;
      ga = dA + A1 * ga;
      const float apt = lane_bcast(apl, t);
      const float ca = quad_sum(live ? gws * wsp[t] + ga * apt : 0.f);
      const float ce = quad_sum(live ? gws * wzc[t] : 0.f);
      const float cb = quad_sum(live ? gwz * wzp[t] : 0.f);
      U.r.red[0][t][qrow] = ca;
      U.r.red[1][t][qrow] = ce;
      U.r.red[2][t][qrow] = cb;
      const int j = t + H - lane;
      const bool wv_ok = src && j >= 0 && j < e;
      U.r.dw[wv_ok ? t * e + j : CH * kWalkWindow] = gwz;
    }
  }
  __builtin_amdgcn_wave_barrier();
  // sums over the quads: lanes 0..31 alpha and eta of step t = lane, lanes 32..63 beta of step lane - 32
  {
    const int t = lane & (CH - 1);
    auto row_sum = [&](int q) {
      const float4* r = reinterpret_cast<const float4*>(&U.r.red[q][t][0]);
      const float4 x0 = r[0], x1 = r[1], x2 = r[2];
      const float x3 = U.r.red[q][t][12];
      return ((x0.x + x0.y) + (x0.z + x0.w)) + ((x1.x + x1.y) + (x1.z + x1.w)) + ((x2.x + x2.y) + (x2.z + x2.w)) + x3;
    };
    if (lane < CH) {
      const float s0 = row_sum(0), s1 = row_sum(1);
      if (t < L) {
        a.ddecay[tb + t0 + t] = from_f32<bf16>(s0);
        a.dlr[tb + t0 + t] = from_f32<bf16>(s1);
      }
    } else {
      const float s0 = row_sum(2);
      if (t < L && g.momentum && a.dbeta) a.dbeta[tb + t0 + t] = from_f32<bf16>(s0);
    }
  }
  // window-weight gradients, written contiguously per chunk
  if (g.gate_mode != GATE_NONE) {
    for (int idx = lane; idx < CH * e; idx += 64) {
      if (idx / e < L) {
        const float v = U.r.dw[idx];
        if (g.gate_mode == GATE_LAG) a.dgate[(tb + t0) * e + idx] = from_f32<bf16>(v);
        else p.dw[(tb + t0) * e + idx] = v;
      }
    }
  }
}

// with_fixup: the launch also runs the segment fixup (valid without token gates, whose gradients
// the fixup forms from the chains' output, and without a buffer_out gradient)
hipError_t launch_scalar_chain(const Geom& g, const BwdPtrs<bf16>& a, const BwdSegPtrs& p, const SegGeom& sg,
                               bool with_fixup, hipStream_t stream) {
  const int nchain = (g.nc + wb::kChainWaves - 1) / wb::kChainWaves;
  hipLaunchKernelGGL(k_scalar_chain, dim3(nchain + (with_fixup ? sg.nseg : 0), g.BH), dim3(64 * wb::kChainWaves), 0,
                     stream, g, a, p, sg, nchain);
  return hipGetLastError();
}

}  // namespace atlas
