// chunk_bwd.hip - reverse walk of the backward pass with every coefficient and the scalar gradients
// formed in the kernel (bf16 inputs, d_k = d_v = 64, window <= 17, no scan_chunk_len clamp, no
// carried buffer).
//
// One workgroup of 8 waves per (segment, row); the segments are the forward's (G chunks of 64
// tokens). The adjoint at each segment end comes from the adjoint aggregates and their scan
// (seg_bwd.hip); the boundary merge and the dS_ref sum are the shared fixup (seg_fixup.h). The
// chunk-start states X_c = (S_c, Z_c) are the forward walk's (bf16, one block per chunk).
//
// Reverse pass, chunk c (targets t = 0 .. 63, sources s = 0 .. 79 at tokens t0 - 16 + s), with
// Lam = (lamS, lamZ) the adjoint of (S, Z) after the chunk's last token:
//   dpsi_t  = S_{t-1}^T dy_t = At S_c^T dy_t + Kt Z_c^T dy_t + sum_s R[s][t] phi_s
//   ddelta_s = sum_t Q[s][t] dy_t + cs_s lamS phi_s + cz_s lamZ phi_s
//   dphi_s  = sum_t R[s][t] psi_t + cs_s lamS^T delta_s + cz_s lamZ^T delta_s + S_ref^T ddelta_s
//   with K[s][t] = phi_s . psi_t, Dd[s][t] = delta_s . dy_t, Wy[s][t] the coefficient of
//   G_s = delta_s phi_s^T in S_{t-1} (the window band times C', C'[r][t] the coefficient of g_r in
//   S_{t-1}), Q = K o Wy, R = Dd o Wy, cs / cz the coefficients of G_s in S / Z at the chunk end;
// the scalar gradients are inner products of the adjoint at t with the state at t - 1, both
//   combinations of a few bases: adjoint bases E_q = dy_q psi_q^T (q > t) and the end adjoint;
//   state bases G_s, S_c, Z_c. With their Gram matrix M on the matrix cores:
//     dalpha_t = <lamS_t, S_{t-1}>,  deta_t = -(beta_t <lamS_t, Z_{t-1}> + <lamS_t, g_t>),
//     dbeta_t = <lamZ_t, Z_{t-1}>,   dw[t][j] = <lamZ_t, G_{t-j}>;
//   then Lam <- T_c^T Lam + sum_t (At, Kt) E_t.
// The halo sources of chunk c are the last 16 tokens of chunk c - 1: their partial gradients stay
// in the registers of the lanes that hold those tokens' rows in the next step.
#include "chunk_common.h"
#include "seg_fixup.h"

namespace atlas {

namespace cpb {
using namespace cp;

constexpr int NTB = 512;

// The walk's arguments, re-read from the kernarg segment where the chunk loop uses them (scalar
// loads through a laundered pointer) instead of being held in scalar registers for the whole walk:
// the loop needs more uniform values than there are scalar registers, and those held would be
// spilled to vector-register lanes and read back with v_readlane on every chunk.
struct CpArgs {
  Geom g;
  BwdPtrs<bf16> a;
  SegGeom sg;
  BwdSegPtrs p;
};
typedef const __attribute__((address_space(4))) CpArgs* CpK;
__device__ __forceinline__ CpK kargs() {
  CpK k = (CpK)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(k));
  return k;
}

// The thread index through an empty asm: values derived from it inside the walk's loops are
// recomputed where they are used instead of being hoisted out of the loop and held in registers
// for its whole length.
__device__ __forceinline__ int fresh_tid() { return launder((int)threadIdx.x); }
#define CPB_FRESH_LANE                                                  \
  const int tid = fresh_tid(), lane = tid & 63, gq = lane >> 4, m = lane & 15; \
  (void)tid; (void)lane; (void)gq; (void)m;
constexpr int NWB = NTB / 64;
constexpr int QP = 88;    // pitch of the Q^T / R^T rows [t][s] (80 sources + 8)
// pitch of the Gram rows [q][s'] (96 state bases: 80 products, S_c, Z_c, zeros; + 8: 52 dwords, so
// that the rows of 16 lanes fall on distinct banks)
constexpr int MQ = 104;
constexpr int QX = CL + 16;   // Gram rows: 64 adjoint bases E_q, then the chunk-end adjoint's partials
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
  // Gram M[q][s'] of adjoint bases q and state bases s' (s' < 80: G_s; 80: S_c; 81: Z_c; rest zero).
  // Rows q < 64: E_q = dy_q psi_q^T. Rows 64 + ct / 68 + ct: lamS / lamZ (the adjoint after the
  // chunk) restricted to the state columns of tile ct (partials summed by the products that read
  // them), their S_c / Z_c entries in rows 64 / 68 only. Rows 72 .. 79 zero.
  alignas(16) bf16 Mt[QX][MQ];
  alignas(16) bf16 Cb[CL][PB];       // C'[r][t]: of g_r in S_{t-1} (r, t chunk-local targets)
  alignas(16) Rows64 DA;              // DA[t][u] = A(u -> t - 1): the decay from token u + 1 to t - 1 (u < t)
  alignas(16) Rows64 BE;              // BE[r][u] = -eta_u B(r -> u) (u >= r): g_r in Z_u, into S_u
  ChunkCoef cc[2];                   // by chunk parity: the chunk in flight and the next one
  float gram[NWB][4];
  // the window band Bd[s][r] = w(r, r + HT - s) (0 <= r + HT - s < e; zero elsewhere): the weight of
  // source s in the window of target r, i.e. of lag j = r + HT - s (w: the lag gate, the token gate
  // of the source, or 1; zero for targets past T)
  alignas(16) BandRows Bd;
};

static_assert(sizeof(BwSm) <= 160 * 1024, "one workgroup per CU: at most 160 KB of LDS");

// register prefetch of one chunk's rows in wave-loads of 8 rows (64 lanes x 16 bytes): wave-load j
// = w + 8 u of wave w. j < 10: phi rows t0 - 16 + 8 j ..; < 20: v rows; < 28: psi rows t0 + ..; < 36:
// dy rows. The kind of a wave-load is uniform over the wave (scalar branches; the rows before token
// 0 read as zeros: their offsets lie outside the buffer resource).
constexpr int WL_R = 2 * SRC / 8 + 2 * CL / 8;   // 36: phi, v, psi, dy
template <int NWL>
struct RowPf { u32x4v v[(NWL + NWB - 1) / NWB]; };

template <int NWL>
__device__ __forceinline__ void rows_load(RowPf<NWL>& pf, int t0, int w) {
  const int lane = fresh_tid() & 63;
  const CpK K = kargs();
  const size_t rb = (size_t)blockIdx.y * K->g.T * D;
  const uint32_t nb = (uint32_t)K->g.T * (D * 2);
  const uint32_t lo = (uint32_t)((lane >> 3) * (D * 2) + (lane & 7) * 16);
  // One load per wave-load with the row tensor chosen by uniform selects: no branches, so the loads
  // are all in flight together (loads in alternative branches writing the same registers would each
  // wait for every load issued before them). Wave-loads past NWL read zeros (an offset out of range).
#pragma unroll
  for (int u = 0; u < (NWL + NWB - 1) / NWB; ++u) {
    const int j = w + NWB * u;
    const bool is_k = j < SRC / 8, is_v = j < 2 * SRC / 8, is_q = j < 2 * SRC / 8 + CL / 8;
    const bf16* base = is_k ? K->a.k : is_v ? K->a.v : is_q ? K->a.q : K->a.dy;
    const int row0 = is_k ? t0 - HT + 8 * j
                   : is_v ? t0 - HT + 8 * (j - SRC / 8)
                   : is_q ? t0 + 8 * (j - 2 * SRC / 8) : t0 + 8 * (j - 2 * SRC / 8 - CL / 8);
    pf.v[u] = bld16(make_rsrc(base + rb, nb), j < NWL ? (uint32_t)(row0 * (D * 2)) + lo : kOob);
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

// the chunk's scalars (waves 0, 1: lane = target) and gates (raw bf16 bits)
struct ScalPf {
  unsigned short al, et, be;
  unsigned short gt[3];
};
// The thread's three window slots i = tid + NTB u (target r = i / e, lag j = i - r e), formed once per
// launch: bits 0-10 rc e + j (rc = min(r, CL - 1)), 11-16 rc, 17-21 j, 22 r < CL. Per chunk the
// gate loads then need no division and no multiply.
struct GateIdx {
  unsigned v[3];
};
__device__ __forceinline__ GateIdx gate_idx(int tid, int e) {
  GateIdx gx;
#pragma unroll
  for (int u = 0; u < 3; ++u) {
    const int i = tid + NTB * u;
    const int r = i / e, j = i - r * e, rc = min(r, CL - 1);
    gx.v[u] = (unsigned)(rc * e + j) | ((unsigned)rc << 11) | ((unsigned)j << 17) | ((r < CL ? 1u : 0u) << 22);
  }
  return gx;
}
static_assert((CL - 1) * EMAX + EMAX - 1 < (1 << 11) && CL <= 64 && EMAX <= 32, "GateIdx fields");

__device__ __forceinline__ void scal_load(ScalPf& p, int t0, const GateIdx& gx) {
  const int tid = fresh_tid();
  const CpK K = kargs();
  const int T = K->g.T, e = K->g.e, gm = K->g.gate_mode;
  const size_t rowbase = (size_t)blockIdx.y * T;
  // Every load is unconditional (clamped index, a valid pointer for absent tensors) and the values
  // are selected afterwards, so that the loads are in flight together (a load under a condition
  // would wait for every load before it).
  // waves 0 and 1 (lane = target): the prefix arrays and the end record are formed from them
  const int ts = t0 + (tid & 63);
  const size_t o = rowbase + min(ts, T - 1);
  const bf16* bsrc = K->g.momentum ? K->a.beta : K->a.decay;
  const unsigned short xa = __builtin_bit_cast(unsigned short, K->a.decay[o]);
  const unsigned short xe = __builtin_bit_cast(unsigned short, K->a.lr[o]);
  const unsigned short xb = __builtin_bit_cast(unsigned short, bsrc[o]);
  // window weight w(r, j) of target r, lag j: the lag gate, the gate of the source token t0 + r - j,
  // or 1; zero for targets past T
  // the row's gates: [T][e] (lag) or [T] (token; none: any valid tensor)
  const bf16* grow = gm == GATE_NONE ? K->a.decay + rowbase : gm == GATE_LAG ? K->a.gate + rowbase * e : K->a.gate + rowbase;
  unsigned short xg[3];
  bool gok[3];
#pragma unroll
  for (int u = 0; u < 3; ++u) {
    const unsigned pk = gx.v[u];
    const int rce = (int)(pk & 0x7ffu), rc = (int)((pk >> 11) & 63u), j = (int)((pk >> 17) & 31u);
    const int tr = t0 + rc;   // the target token (clamped row)
    // lag: (tr, j) = element tr e + j, clamped into the row (a target past T is masked below);
    // token: the gate of source tr - j, clamped into the row
    const int gi = gm == GATE_LAG ? min(t0 * e + rce, T * e - 1) : min(max(tr - j, 0), T - 1);
    xg[u] = __builtin_bit_cast(unsigned short, grow[gi]);
    gok[u] = (pk >> 22) != 0u && tr < T && (gm != GATE_TOKEN || tr - j >= 0);
  }
  const bool sok = tid < 128 && ts < T;
  p.al = sok ? xa : (unsigned short)0x3f80;   // 1, 0, 1: the identity past T
  p.et = sok ? xe : (unsigned short)0;
  p.be = sok ? (K->g.momentum ? xb : (unsigned short)0) : (unsigned short)0x3f80;
#pragma unroll
  for (int u = 0; u < 3; ++u) p.gt[u] = gok[u] ? (gm == GATE_NONE ? (unsigned short)0x3f80 : xg[u]) : (unsigned short)0;
}
__device__ __forceinline__ void gates_store(const ScalPf& p, const GateIdx& gx, BwSm& sm) {
#pragma unroll
  for (int u = 0; u < 3; ++u) {
    const unsigned pk = gx.v[u];
    if ((pk >> 22) != 0u) {   // r < CL (then r = rc)
      const int r = (int)((pk >> 11) & 63u), j = (int)((pk >> 17) & 31u);
      sm.Bd[r + HT - j][r] = __builtin_bit_cast(bf16, p.gt[u]);
    }
  }
}

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

// Sum over the 64 lanes, in every lane (DPP row sums, then the cross-row swaps).
__device__ __forceinline__ float wave_sum(float x) { return xsum_rows(row_sum16(x)); }

__device__ __forceinline__ unsigned pk(float a, float b) { return pack_bf16x2(a, b); }
// v stored at byte offset off (32-bit) from a uniform base: one store with a scalar base and a 32-bit
// vector offset instead of per-lane 64-bit address arithmetic
template <typename B, typename V>
__device__ __forceinline__ void st_at(B* base, uint32_t off, V v) {
  *reinterpret_cast<V*>(reinterpret_cast<unsigned char*>(base) + off) = v;
}
__device__ __forceinline__ float lo16(unsigned u) { return __builtin_bit_cast(float, u << 16); }
__device__ __forceinline__ float hi16(unsigned u) { return __builtin_bit_cast(float, u & 0xffff0000u); }

}  // namespace cpb

using namespace cpb;

template <bool MAPE, bool MOM>
__global__ __launch_bounds__(NTB) void k_cp_bwd(const CpArgs A) {
  const Geom& g = A.g;
  const BwdPtrs<bf16>& a = A.a;
  const SegGeom& sg = A.sg;
  const BwdSegPtrs& p = A.p;
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
  const size_t DD = (size_t)D * D;

  // chunk-start states saved by the forward walk (walk_common.h fragment layout), one block per
  // 64-token chunk of the row: this lane's slice X[16 q4 + 4 gq + r][16 kt + m] (kt = 2 hf + j) is
  // one 8-byte half of fragment (kt, q4 >> 1)
  auto xs_load = [&](int c, unsigned (&xv)[8]) {
    const CpK K = kargs();
    const unsigned char* blk = reinterpret_cast<const unsigned char*>(K->p.rw) + ((size_t)bh * K->g.nc + c) * kStateBlk;
    const int ln = fresh_tid() & 63;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const uint32_t o = frag_off(2 * hf + jj, q4 >> 1, ln) + (q4 & 1) * 8;
      const uint2 s2 = *reinterpret_cast<const uint2*>(blk + o);
      const uint2 z2 = *reinterpret_cast<const uint2*>(blk + kStateBytes + o);
      xv[4 * jj + 0] = s2.x; xv[4 * jj + 1] = s2.y;
      xv[4 * jj + 2] = MOM ? z2.x : 0u; xv[4 * jj + 3] = MOM ? z2.y : 0u;
    }
  };

  // the last chunk's loads go out first: its scalars, rows and state slice are in flight while
  // S_ref, the segment-end adjoint and the zeroed LDS tables are set up
  RowPf<WL_R> pf;
  ScalPf sp;
  unsigned xn[8];   // the next chunk's state slice, in flight with its rows
  const GateIdx gxi = gate_idx(tid, g.e);
  scal_load(sp, (c_end - 1) * CL, gxi);
  rows_load<WL_R>(pf, (c_end - 1) * CL, w);
  xs_load(c_end - 1, xn);

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
  // the Gram's entries that are never written stay zero
  for (int i = tid; i < QX * MQ / 2; i += NTB) reinterpret_cast<unsigned*>(&sm.Mt[0][0])[i] = 0u;
  __syncthreads();

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

  // the last chunk's record and prefix arrays (every later chunk's are formed one step ahead)
  if (w == 0) chunk_prefix(bf(sp.al), bf(sp.et), bf(sp.be), lane, sm.cc[(c_end - c_begin - 1) & 1]);
  if (w == 1) chunk_end_scan(g.T, bf(sp.al), bf(sp.et), bf(sp.be), (c_end - 1) * CL, lane, sm.cc[(c_end - c_begin - 1) & 1]);
  __syncthreads();
  gen_tables<MOM>(sm.cc[(c_end - c_begin - 1) & 1], sm.DA, sm.BE, tid);   // (every later chunk's: in R4 before it)
#pragma unroll 1
  for (int cr = c_end - c_begin - 1; cr >= 0; --cr) {
    CPB_FRESH_LANE
    // the wave's role, recomputed each chunk (conditions derived from it are not held across the loop)
    ChunkCoef& kc = sm.cc[cr & 1];   // this chunk's record and prefix arrays (formed one step ahead)
    const int c = c_begin + cr;
    const int t0 = c * CL;
    // this wave's slice of X_c (for the Grams and the LDS copy)
    unsigned xc[8];
#pragma unroll
    for (int v = 0; v < 8; ++v) xc[v] = xn[v];
    const bool seg_last = c == c_end - 1, seg_first = c == c_begin;
    const bool interior = !seg_last && !seg_first;   // uniform: the stores take no per-row tests
    // ---- R0: stage the chunk
    __syncthreads();
    rows_store<MAPE, WL_R>(pf, sm, g.map_deg, w);
    gates_store(sp, gxi, sm);
    // the next chunk's scalars, early: waves 0, 1 form its record and prefix arrays at the end of R4
    scal_load(sp, c > c_begin ? t0 - CL : t0, gxi);   // unconditional (see the rows' prefetch in R3)
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

    // ---- R1: delta (in place of v), the factors of C', the end coefficients, the Grams' end rows
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
      const bf16x8 fbe0 = frag_row_l(&sm.BE[0][0], PB, 16 * q4, 0, lane);
      const bf16x8 fbe1 = frag_row_l(&sm.BE[0][0], PB, 16 * q4, 32, lane);
#pragma unroll
      for (int j = 0; j < 2; ++j) {   // C'[r][t] = sum_u BE[r][u] DA[t][u]: tiles (q4, 2 hf + j)
        const int tt = 2 * hf + j;
        f32x4 acc = zero4();
        acc = mma_bf16(fbe0, frag_row_l(&sm.DA[0][0], PB, 16 * tt, 0, lane), acc);
        acc = mma_bf16(fbe1, frag_row_l(&sm.DA[0][0], PB, 16 * tt, 32, lane), acc);
#pragma unroll
        for (int r = 0; r < 4; ++r) sm.Cb[16 * q4 + 4 * gq + r][16 * tt + m] = static_cast<bf16>(acc[r]);
      }
      chunk_end_sources(g, sm.Bd, kc, tid - 256);   // threads 256 .. 335: cs, cz of the chunk's sources
      if (tid < 4) {   // <lamS, S_c>, <lamS, Z_c>, <lamZ, S_c>, <lamZ, Z_c> into the end rows
        float gsum = 0.f;
#pragma unroll
        for (int u = 0; u < NWB; ++u) gsum += sm.gram[u][tid];
        sm.Mt[tid < 2 ? CL : CL + 4][SRC + (tid & 1)] = static_cast<bf16>(gsum);
      }
    }
    __syncthreads();
    // ---- R2: t-phase (waves 0-3) | end terms of ddelta / dphi (waves 4-7)
    // the end terms (waves 4-7), bf16 pairs in the accumulator layout, used in R3 / R4
    unsigned edr[SRC / 16][2], efr[SRC / 16][2];
    if (hf == 0) {
      CPB_FRESH_LANE
      const int tt = q4;
      const int t = 16 * tt + m;
      const CpK K = kargs();
      const size_t rb = (size_t)bh * K->g.T * D;
      const uint32_t nb = (uint32_t)K->g.T * (D * 2);
      const rsrc_t rdq = make_rsrc(K->a.dq + rb, nb);
      // C' as the k-major operand over the targets r (lane row t): shared by every source tile
      const bf16x8 fcb0 = frag_tr_l(&sm.Cb[0][0], PB, 16 * tt, 0, lane);
      const bf16x8 fcb1 = frag_tr_l(&sm.Cb[0][0], PB, 16 * tt, 32, lane);
      // the targets' psi and dy rows, read once for every source tile and the dpsi products
      bf16x8 fps[2], fdy[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        fps[q] = frag_row_l(&sm.psi[0][0], PB, 16 * tt, 32 * q, lane);
        fdy[q] = frag_row_l(&sm.dy[0][0], PB, 16 * tt, 32 * q, lane);
      }
      f32x4 Rr[SRC / 16];
#pragma unroll
      for (int st = 0; st < SRC / 16; ++st) {
        f32x4 kq = zero4(), dd = zero4(), wy = zero4();
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          kq = mma_bf16(frag_row_l(&sm.phi[0][0], PB, 16 * st, 32 * q, lane), fps[q], kq);
          dd = mma_bf16(frag_row_l(&sm.vd[0][0], PB, 16 * st, 32 * q, lane), fdy[q], dd);
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
      const float At = kc.At[t], Kt = kc.Kt[t];
      float fS = 0.f, fZ = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        f32x4 di = zero4(), ds = zero4(), dz = zero4();
        di = mma_bf16(tr_pair_l<true>(&sm.phi[0][0], PB, 0, 16 * kt, lane), fr0, di);
        di = mma_bf16(tr_pair_l<true>(&sm.phi[0][0], PB, 1, 16 * kt, lane), fr1, di);
        di = mma_bf16(tr_pair_l<false>(&sm.phi[0][0], PB, 2, 16 * kt, lane), fr2, di);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          ds = mma_bf16(frag_row_l(&sm.XS[0][0][0], PB, 16 * kt, 32 * q, lane), fdy[q], ds);
          dz = mma_bf16(frag_row_l(&sm.XS[1][0][0], PB, 16 * kt, 32 * q, lane), fdy[q], dz);
        }
        const float4 ps = lds_bf16x4(&sm.psi[t][16 * kt + 4 * gq]);
        fS += ps.x * ds[0] + ps.y * ds[1] + ps.z * ds[2] + ps.w * ds[3];
        fZ += ps.x * dz[0] + ps.y * dz[1] + ps.z * dz[2] + ps.w * dz[3];
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = di[r] + At * ds[r] + Kt * dz[r];
        if constexpr (MAPE) {
          const u32x2v raw = bld8(make_rsrc(K->a.q + rb, nb), (uint32_t)(((t0 + t) * D + 16 * kt + 4 * gq) * 2));
          const int deg = K->g.map_deg;
          o[0] *= poly_map_grad(lo16(raw[0]), deg); o[1] *= poly_map_grad(hi16(raw[0]), deg);
          o[2] *= poly_map_grad(lo16(raw[1]), deg); o[3] *= poly_map_grad(hi16(raw[1]), deg);
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
      // transposed tiles: rows i (or k) = 16 ct + 4 gq + r, columns s = 16 st + m
      const int ct = q4;
      bf16x8 ones;
#pragma unroll
      for (int e = 0; e < 8; ++e) ones[e] = static_cast<bf16>(1.f);
      // the adjoint's operands of this wave's rows / columns, read once for every source tile
      bf16x8 fls[2], flz[2], fks[2], fkz[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        fls[q] = frag_tr_l(&sm.XL[0][0][0], PB, 16 * ct, 32 * q, lane);
        flz[q] = frag_tr_l(&sm.XL[1][0][0], PB, 16 * ct, 32 * q, lane);
        fks[q] = frag_row_l(&sm.XL[0][0][0], PB, 16 * ct, 32 * q, lane);
        fkz[q] = frag_row_l(&sm.XL[1][0][0], PB, 16 * ct, 32 * q, lane);
      }
#pragma unroll
      for (int st = 0; st < SRC / 16; ++st) {
        f32x4 es = zero4(), ez = zero4(), fs = zero4(), fz = zero4();
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const bf16x8 fp = frag_row_l(&sm.phi[0][0], PB, 16 * st, 32 * q, lane);
          es = mma_bf16(fls[q], fp, es);   // (lamS phi_s)[i]
          ez = mma_bf16(flz[q], fp, ez);
          const bf16x8 fd = frag_row_l(&sm.vd[0][0], PB, 16 * st, 32 * q, lane);
          fs = mma_bf16(fks[q], fd, fs);   // (lamS^T delta_s)[k]
          fz = mma_bf16(fkz[q], fd, fz);
        }
        // hS[s] = delta_s . (lamS phi_s): this wave's 16 rows i summed on the matrix cores (every
        // output row holds the column sums); the four column tiles are the Gram's end-row partials
        const float4 dl = lds_bf16x4(&sm.vd[16 * st + m][16 * ct + 4 * gq]);
        const float dv4[4] = {dl.x, dl.y, dl.z, dl.w};
        f32x4 ps, pz;
#pragma unroll
        for (int r = 0; r < 4; ++r) { ps[r] = dv4[r] * es[r]; pz[r] = dv4[r] * ez[r]; }
        const f32x4 hs = mma_bf16(ones, pack_frag(ps, zero4()), zero4());
        const f32x4 hz = mma_bf16(ones, pack_frag(pz, zero4()), zero4());
        if (gq == 0) {
          sm.Mt[CL + ct][16 * st + m] = static_cast<bf16>(hs[0]);
          sm.Mt[CL + 4 + ct][16 * st + m] = static_cast<bf16>(hz[0]);
        }
        const float cs = kc.co[R_CS + 16 * st + m], cz = kc.co[R_CZ + 16 * st + m];
        edr[st][0] = pk(cs * es[0] + cz * ez[0], cs * es[1] + cz * ez[1]);
        edr[st][1] = pk(cs * es[2] + cz * ez[2], cs * es[3] + cz * ez[3]);
        efr[st][0] = pk(cs * fs[0] + cz * fz[0], cs * fs[1] + cz * fz[1]);
        efr[st][1] = pk(cs * fs[2] + cz * fz[2], cs * fs[3] + cz * fz[3]);
      }
    }
    __syncthreads();

    // The window gradients dw[t][j] = <lamZ_t, G_{t-j}> = (Km M)[t][t + HT - j] of the wave's
    // targets t = 16 q4 + 4 gq + r over state-base tile q4 + h (the band of t spans tiles q4 and
    // q4 + 1): tile 0 in R3 by waves 4-7, ahead of their ddelta (so that its LDS reads do not queue
    // behind the ddelta stores), tile 1 in R4 by waves 0-3 (Mt, Cb and the record stay unchanged
    // until the next chunk's R0).
    auto dw_tile = [&](int h) {
      CPB_FRESH_LANE
      const CpK Kw = kargs();
      const int gm = Kw->g.gate_mode, ne = Kw->g.e, T = Kw->g.T;
      if (gm == GATE_NONE) return;
      // outputs of row bh: lag gates bf16 [T][e], or the per-(target, lag) fp32 terms of token gates
      bf16* const dg_row = Kw->a.dgate + (size_t)bh * T * ne;
      float* const dw_row = Kw->p.dw + (size_t)bh * T * ne;
      const int tt = q4, tl = 16 * tt + m, sp = tt + h;
      const float cgs = kc.co[R_GS + tl], cgz = kc.co[R_GZ + tl];
      bf16x8 kme;   // Km over the end rows (k = 64 + 8 gq + e): cgS on the lamS partials, cgZ on lamZ's
#pragma unroll
      for (int e = 0; e < 8; ++e) kme[e] = static_cast<bf16>(gq == 0 ? (e < 4 ? cgs : cgz) : 0.f);
      f32x4 rz = zero4();
      rz = mma_bf16(frag_row_l(&sm.Cb[0][0], PB, 16 * tt, 0, lane), frag_tr_l(&sm.Mt[0][0], MQ, 16 * sp, 0, lane), rz);
      rz = mma_bf16(frag_row_l(&sm.Cb[0][0], PB, 16 * tt, 32, lane), frag_tr_l(&sm.Mt[0][0], MQ, 16 * sp, 32, lane), rz);
      // rows 64 .. 79 only (lanes 0 .. 31 address them; the others' k slots carry zero weights)
      const bf16x8 me = frag_tr_l(&sm.Mt[0][0], MQ, 16 * sp, 64 - 16 * (gq >> 1), lane);
      rz = mma_bf16(kme, gq < 2 ? me : zero_frag(), rz);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * tt + 4 * gq + r, sq = 16 * sp + m;
        const int jb = t + HT - sq;
        if (jb >= 0 && jb < ne && t0 + t < T) {
          const uint32_t o = (uint32_t)((t0 + t) * ne + jb);
          if (gm == GATE_LAG) st_at(dg_row, o * 2, static_cast<bf16>(rz[r]));
          else st_at(dw_row, o * 4, rz[r]);
        }
      }
    };

    // the next chunk's rows and state slice in flight from here to its R0. Unconditional (the
    // segment's first chunk loads itself again, never used): a load under a condition would make
    // the next wait on any earlier load wait for every load issued so far.
    {
      const int cn = c > c_begin ? c - 1 : c;
      rows_load<WL_R>(pf, cn * CL, w);
      xs_load(cn, xn);
    }
    // ---- R3: ddelta, dv (waves 4-7) | scalar gradients (waves 0-3)
    if (hf == 1) {
      CPB_FRESH_LANE
      dw_tile(0);
      const int ct = q4;
      const CpK K = kargs();
      const size_t rowbase = (size_t)bh * K->g.T;
      float cin[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) cin[r] = cdv[r];
      bf16x8 fdt[2];   // dy^T rows of this wave's columns, read once for every source tile
#pragma unroll
      for (int q = 0; q < 2; ++q) fdt[q] = frag_tr_l(&sm.dy[0][0], PB, 16 * ct, 32 * q, lane);
#pragma unroll
      for (int st = 0; st < SRC / 16; ++st) {
        f32x4 acc;
        {
          const unsigned e0 = edr[st][0], e1 = edr[st][1];
          acc[0] = lo16(e0); acc[1] = hi16(e0); acc[2] = lo16(e1); acc[3] = hi16(e1);
        }
#pragma unroll
        for (int q = 0; q < 2; ++q)   // ddelta^T[i][s] = sum_t dy[t][i] Q[s][t] (+ the end terms)
          acc = mma_bf16(fdt[q], frag_tr_l(&sm.Qt[0][0], QP, 16 * st, 32 * q, lane), acc);
        // this lane: source s = 16 st + m, columns col0 .. col0 + 3
        const int s = 16 * st + m, pp = t0 - HT + s, col0 = 16 * ct + 4 * gq;
        store4<bf16>(&sm.vd[s][col0], acc[0], acc[1], acc[2], acc[3]);
        float val[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) val[r] = -acc[r];
        if (interior) {   // no segment boundary, no tail rows, every row < T
          if (st == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) cdv[r] = val[r];
          } else {
            if (st == SRC / 16 - 1)
#pragma unroll
              for (int r = 0; r < 4; ++r) val[r] += cin[r];
            st_at(K->a.dv + rowbase * D, (uint32_t)((pp * D + col0) * 2), make_uint2(pk(val[0], val[1]), pk(val[2], val[3])));
          }
        } else if (st == 0) {   // halo rows: partial for the previous chunk (or the previous segment)
          if (seg_first) {
            if (seg > 0 && s >= HT - H)
              st_at(part_row(K->p.halo_part, bh, K->sg.nseg, seg, H), (uint32_t)(((s - (HT - H)) * (2 * D) + col0) * 4),
                    make_float4(val[0], val[1], val[2], val[3]));
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) cdv[r] = val[r];
          }
        } else if (pp < K->g.T) {
          if (st == SRC / 16 - 1 && !seg_last)
#pragma unroll
            for (int r = 0; r < 4; ++r) val[r] += cin[r];
          if (pp >= tail0)
            st_at(part_row(K->p.tail_part, bh, K->sg.nseg, seg, H), (uint32_t)(((pp - tail0) * (2 * D) + col0) * 4),
                  make_float4(val[0], val[1], val[2], val[3]));
          else
            st_at(K->a.dv + rowbase * D, (uint32_t)((pp * D + col0) * 2), make_uint2(pk(val[0], val[1]), pk(val[2], val[3])));
        }
      }
    } else {
      CPB_FRESH_LANE
      const int tt = q4;
      // The scalar gradients of target t = 16 tt + (lane & 15):
      //   dalpha_t = <lamS_t, S_{t-1}>, deta_t = -(beta_t <lamS_t, Z_{t-1}> + <lamS_t, g_t>),
      //   dbeta_t = <lamZ_t, Z_{t-1}>, dw[t][j] = <lamZ_t, G_{t-j}>,
      // with lamS_t = sum_q Am[t][q] E_q (q over the adjoint bases, the end rows included) and the
      // total lamZ_t = sum_q Km[t][q] E_q; S_{t-1} = sum_s' Wy~[s'][t] X_s', Z_{t-1} = sum_s' Wz~[s'][t] X_s'
      // over the state bases X_s'. So dalpha_t = sum_q Am[t][q] (M Wy~)[q][t]: the products M Wy~,
      // M Wz~ and M Band (for <lamS_t, g_t>) on the matrix cores, then one weighted sum over q.
      const bf16x8 fcb0 = frag_tr_l(&sm.Cb[0][0], PB, 16 * tt, 0, lane);
      const bf16x8 fcb1 = frag_tr_l(&sm.Cb[0][0], PB, 16 * tt, 32, lane);
      // Wy~ = Band C' (+ At, Kt in rows 80, 81) and Wz~ = Band B' (+ B1 in row 81): tiles of 16 state
      // bases (rows) by this wave's targets (columns), packed in pairs as the k-chained operands
      bf16x8 wyp[3], wzp[3];
      {
        const bf16x8 fz0 = gen_zcoef<MOM>(kc.lb, 16 * tt + m, 0, lane);
        const bf16x8 fz1 = gen_zcoef<MOM>(kc.lb, 16 * tt + m, 1, lane);
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          f32x4 y[2], z[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int st = 2 * i + h;
            y[h] = zero4();
            z[h] = zero4();
            // the band of source tile st meets k half 0 for st <= 2, half 1 for 2 <= st <= 4
            if (st <= 2) {
              const bf16x8 fb = frag_row_l(&sm.Bd[0][0], PB, 16 * st, 0, lane);
              y[h] = mma_bf16(fb, fcb0, y[h]);
              z[h] = mma_bf16(fb, fz0, z[h]);
            }
            if (st >= 2 && st <= 4) {
              const bf16x8 fb = frag_row_l(&sm.Bd[0][0], PB, 16 * st, 32, lane);
              y[h] = mma_bf16(fb, fcb1, y[h]);
              z[h] = mma_bf16(fb, fz1, z[h]);
            }
          }
          if (i == 2 && gq == 0) {   // rows 80 (S_c), 81 (Z_c) of tile 5
            const int t = 16 * tt + m;
            y[1][0] = kc.At[t];
            y[1][1] = kc.Kt[t];
            z[1][1] = kc.B1[t];
          }
          wyp[i] = pack_frag(y[0], y[1]);
          wzp[i] = pack_frag(z[0], z[1]);
        }
      }
      // Band as the k-chained operand over the state bases (rows 80 .. 95 zero)
      const bf16x8 bdp0 = tr_pair_l<true>(&sm.Bd[0][0], PB, 0, 16 * tt, lane);
      const bf16x8 bdp1 = tr_pair_l<true>(&sm.Bd[0][0], PB, 1, 16 * tt, lane);
      const bf16x8 bdp2 = tr_pair_l<false>(&sm.Bd[0][0], PB, 2, 16 * tt, lane);
      const int tl = 16 * tt + m;   // this lane's target (accumulator column)
      const float lat = kc.la[tl];
      const float aend = __builtin_amdgcn_exp2f(kc.la[CL - 1] - lat);
      const float cgs = kc.co[R_GS + tl], cgz = kc.co[R_GZ + tl];
      float al = 0.f, ea = 0.f, eb = 0.f, bt = 0.f;
#pragma unroll
      for (int qt = 0; qt < QX / 16; ++qt) {
        // M rows q = 16 qt + (lane & 15) as the k-chained A operand over s'
        bf16x8 mf[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          const bf16* mrow = &sm.Mt[16 * qt + m][32 * i + 4 * gq];
          const uint2 lo = *reinterpret_cast<const uint2*>(mrow);
          const uint2 hi = *reinterpret_cast<const uint2*>(mrow + 16);
          mf[i] = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
        }
        f32x4 py = zero4(), pz = zero4(), mb = zero4();
        py = mma_bf16(mf[0], wyp[0], py); py = mma_bf16(mf[1], wyp[1], py); py = mma_bf16(mf[2], wyp[2], py);
        pz = mma_bf16(mf[0], wzp[0], pz); pz = mma_bf16(mf[1], wzp[1], pz); pz = mma_bf16(mf[2], wzp[2], pz);
        mb = mma_bf16(mf[0], bdp0, mb); mb = mma_bf16(mf[1], bdp1, mb); mb = mma_bf16(mf[2], bdp2, mb);
        // adjoint coefficients of the rows q = 16 qt + 4 gq + r for target tl
        float am[4], km[4];
        if (qt < CL / 16) {
          const int q0 = 16 * qt + 4 * gq;
          // Am[t][q] = A(t -> q - 1) = DA[q][t] (zero for q <= t): rows q0 .. q0 + 3 of column tl
          const s16x4 av = tr4_l(&sm.DA[0][0], PB, 16 * qt, 16 * tt, lane);
          const float4 kq = lds_bf16x4(&sm.Cb[tl][q0]);
          const float kv[4] = {kq.x, kq.y, kq.z, kq.w};
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            am[r] = bf((unsigned short)av[r]);
            km[r] = kv[r];
          }
        } else {   // the end rows: lamS partials (64 .. 67), lamZ partials (68 .. 71)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            am[r] = gq == 0 ? aend : 0.f;
            km[r] = gq == 0 ? cgs : (gq == 1 ? cgz : 0.f);
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          al += am[r] * py[r];
          ea += am[r] * pz[r];
          eb += am[r] * mb[r];
          bt += km[r] * pz[r];
        }
      }
      al = xsum_rows(al);
      ea = xsum_rows(ea);
      eb = xsum_rows(eb);
      bt = xsum_rows(bt);
      const CpK K = kargs();
      if (gq == 0 && t0 + tl < K->g.T) {
        const uint32_t o = (uint32_t)(t0 + tl) * 2;
        const size_t rowbase = (size_t)bh * K->g.T;
        st_at(K->a.ddecay + rowbase, o, static_cast<bf16>(al));
        st_at(K->a.dlr + rowbase, o, static_cast<bf16>(-(kc.be[tl] * ea + eb)));
        if (MOM) st_at(K->a.dbeta + rowbase, o, static_cast<bf16>(bt));
      }
      // the next chunk's record and prefix arrays, from the scalars fetched in R0 (the other buffer:
      // this chunk's is still read in R4 and R5)
      if (c > c_begin) {
        if (w == 0) chunk_prefix(bf(sp.al), bf(sp.et), bf(sp.be), lane, sm.cc[(cr - 1) & 1]);
        if (w == 1) chunk_end_scan(K->g.T, bf(sp.al), bf(sp.et), bf(sp.be), t0 - CL, lane, sm.cc[(cr - 1) & 1]);
      }
    }
    __syncthreads();

    // ---- R4: dphi, dk (waves 4-7) | dS_ref partial (waves 0-3)
    if (hf == 1) {
      CPB_FRESH_LANE
      const int ct = q4;
      const CpK K = kargs();
      const size_t rowbase = (size_t)bh * K->g.T;
      float cin[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) cin[r] = cdk[r];
      bf16x8 fpt[2];   // psi^T rows of this wave's columns, read once for every source tile
#pragma unroll
      for (int q = 0; q < 2; ++q) fpt[q] = frag_tr_l(&sm.psi[0][0], PB, 16 * ct, 32 * q, lane);
#pragma unroll
      for (int st = 0; st < SRC / 16; ++st) {
        f32x4 acc;
        {
          const unsigned e0 = efr[st][0], e1 = efr[st][1];
          acc[0] = lo16(e0); acc[1] = hi16(e0); acc[2] = lo16(e1); acc[3] = hi16(e1);
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {   // dphi^T[k][s] = sum_t psi[t][k] R[s][t] + (S_ref^T ddelta_s)[k] (+ end terms)
          acc = mma_bf16(fpt[q], frag_tr_l(&sm.Rt[0][0], QP, 16 * st, 32 * q, lane), acc);
          acc = mma_bf16(sreft[q], frag_row_l(&sm.vd[0][0], PB, 16 * st, 32 * q, lane), acc);
        }
        const int s = 16 * st + m, pp = t0 - HT + s, col0 = 16 * ct + 4 * gq;
        float val[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) val[r] = acc[r];
        auto store_dk = [&](float (&v)[4]) {
          if constexpr (MAPE) {
            const u32x2v raw =
                bld8(make_rsrc(K->a.k + rowbase * D, (uint32_t)K->g.T * (D * 2)), (uint32_t)((pp * D + col0) * 2));
            const int deg = K->g.map_deg;
            v[0] *= poly_map_grad(lo16(raw[0]), deg); v[1] *= poly_map_grad(hi16(raw[0]), deg);
            v[2] *= poly_map_grad(lo16(raw[1]), deg); v[3] *= poly_map_grad(hi16(raw[1]), deg);
          }
          st_at(K->a.dk + rowbase * D, (uint32_t)((pp * D + col0) * 2), make_uint2(pk(v[0], v[1]), pk(v[2], v[3])));
        };
        if (interior) {
          if (st == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) cdk[r] = val[r];
          } else {
            if (st == SRC / 16 - 1)
#pragma unroll
              for (int r = 0; r < 4; ++r) val[r] += cin[r];
            store_dk(val);
          }
        } else if (st == 0) {
          if (seg_first) {
            if (seg > 0 && s >= HT - H)
              st_at(part_row(K->p.halo_part, bh, K->sg.nseg, seg, H), (uint32_t)(((s - (HT - H)) * (2 * D) + D + col0) * 4),
                    make_float4(val[0], val[1], val[2], val[3]));
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) cdk[r] = val[r];
          }
        } else if (pp < K->g.T) {
          if (st == SRC / 16 - 1 && !seg_last)
#pragma unroll
            for (int r = 0; r < 4; ++r) val[r] += cin[r];
          if (pp >= tail0)
            st_at(part_row(K->p.tail_part, bh, K->sg.nseg, seg, H), (uint32_t)(((pp - tail0) * (2 * D) + D + col0) * 4),
                  make_float4(val[0], val[1], val[2], val[3]));
          else
            store_dk(val);
        }
      }
    } else {
      CPB_FRESH_LANE
      // ddelta^T of this wave's rows over the source slots, read once for the four column tiles
      const bf16x8 fv0 = tr_pair_l<true>(&sm.vd[0][0], PB, 0, 16 * q4, lane);
      const bf16x8 fv1 = tr_pair_l<true>(&sm.vd[0][0], PB, 1, 16 * q4, lane);
      const bf16x8 fv2 = tr_pair_l<false>(&sm.vd[0][0], PB, 2, 16 * q4, lane);
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        f32x4 acc = zero4();
        acc = mma_bf16(fv0, tr_pair_l<true>(&sm.phi[0][0], PB, 0, 16 * kt, lane), acc);
        acc = mma_bf16(fv1, tr_pair_l<true>(&sm.phi[0][0], PB, 1, 16 * kt, lane), acc);
        acc = mma_bf16(fv2, tr_pair_l<false>(&sm.phi[0][0], PB, 2, 16 * kt, lane), acc);
#pragma unroll
        for (int r = 0; r < 4; ++r) dsr[kt][r] += acc[r];
      }
      dw_tile(1);
    }
    // the next chunk's C' factors, from its prefix arrays (formed in R3; this chunk's tables were last
    // read in R3)
    if (c > c_begin) gen_tables<MOM>(sm.cc[(cr - 1) & 1], sm.DA, sm.BE, fresh_tid());

    // ---- R5: the adjoint at the chunk start
    {
      CPB_FRESH_LANE
      const float ta = kc.co[R_TR], tk = kc.co[R_TR + 1], tb = kc.co[R_TR + 2];
      f32x4 dS[2], dZ[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) { dS[j] = zero4(); dZ[j] = zero4(); }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const bf16x8 fy = tr_pair_l<true>(&sm.dy[0][0], PB, q, 16 * q4, lane);
        const float4 ahi = *reinterpret_cast<const float4*>(&kc.At[32 * q + 4 * gq]);
        const float4 alo = *reinterpret_cast<const float4*>(&kc.At[32 * q + 16 + 4 * gq]);
        const float4 khi = *reinterpret_cast<const float4*>(&kc.Kt[32 * q + 4 * gq]);
        const float4 klo = *reinterpret_cast<const float4*>(&kc.Kt[32 * q + 16 + 4 * gq]);
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

// The chunk-start states k_cp_bwd reads: saved by the forward walk (walk_fwd.hip), one block per
// 64-token chunk of every row.
size_t chunk_bwd_states_bytes(const Geom& g) { return (size_t)g.BH * g.nc * kStateBlk; }

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
  const CpArgs A{g, a, sg, p};
  if (mape) {
    if (g.momentum) hipLaunchKernelGGL((k_cp_bwd<true, true>), grid, dim3(NTB), smem, stream, A);
    else hipLaunchKernelGGL((k_cp_bwd<true, false>), grid, dim3(NTB), smem, stream, A);
  } else {
    if (g.momentum) hipLaunchKernelGGL((k_cp_bwd<false, true>), grid, dim3(NTB), smem, stream, A);
    else hipLaunchKernelGGL((k_cp_bwd<false, false>), grid, dim3(NTB), smem, stream, A);
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
