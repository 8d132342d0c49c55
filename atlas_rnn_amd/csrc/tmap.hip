// tmap.hip - the tensor polynomial feature map, fused (forward and backward), bf16 in / fp32 accumulate.
//
//   phi = [x; vec(x x^T)] P,   x [N, D],  P [D + D*D, M]        (rnn_memory.py:125-130, the 'tensor'
//                                                                 mode of PolynomialFeatureMap)
// Neither direction materialises the [N, D + D*D] Kronecker features:
//
// forward  (k_tmap_fwd): one GEMM over K = D + D*D in blocks of D: block 0 is x itself, block a + 1
//   the row a of x x^T, i.e. x_a * x. The x-side MFMA operand of a block is formed in registers from
//   the token's x values (x_a from LDS, x_b held per lane), the P-side operand (P^T staged in LDS,
//   double buffered, one barrier per block) is shared by the waves. The accumulator is phi^T, so each
//   lane stores four consecutive features of one token.
//
// backward (k_tmap_bwd): with G[n, a, b] = sum_j dphi[n, j] P[D + D a + b, j] (P's rows are the
//   k operand; dphi stays in registers for the whole launch),
//     dx[n, c] = sum_j dphi[n, j] P[c, j] + sum_b G[n, c, b] x[n, b] + sum_a G[n, a, c] x[n, a].
//   The block of row a yields G[., a, .] as matrix-core tiles; the third term accumulates in the
//   owning lanes (x[n, a] is one value per lane), the second is a sum over b across the tile (in lane
//   and over the four lane rows) written to an LDS table t1[half][n][a] and added at the end.
//
// An elementwise polynomial of degree deg after the projection (phi -> sum_{i=1..deg} phi^i, the
// BASELINE C4 composition) is applied in the forward's epilogue on the fp32 accumulator, which then
// also stores the projection itself (pre); the backward scales dphi by the map's derivative at pre
// as it loads dphi.
//
// Token tiles of 128 rows; rows past N load zeros and their stores are dropped (buffer range checks).
#include <type_traits>

#include "mem_common.h"
#include "walk_common.h"

namespace atlas {

namespace tm {
constexpr int TN = 128;   // tokens per workgroup
// Packed order of the symmetrised table's blocks at d = 64 (zero where b < a), by 32-wide k-steps:
// blocks 0 .. 16 (the linear rows, rows a = 0 .. 15) over both k-steps b in [0, 64); blocks 17 .. 48
// (rows 16 .. 47) over the upper k-step b in [32, 64); then eight quads kPackQuad + q, each four
// 16-column pieces of rows a0 .. a0 + 3 (two per k-step): b in [16, 32) of rows 16 .. 31 (q < 4) and
// b in [48, 64) of rows 48 .. 63 (q >= 4), a0 = 16 + 4 q or 48 + 4 (q - 4). 82 k-steps in all
// instead of 98 with whole upper k-steps for rows 32 .. 63.
constexpr int kPackQuad = 49;
constexpr int kNPack = kPackQuad + 8;
}

// ---------------------------------------------------------------------------------------------
// forward: waves = 4 (token groups of 32) x M / FG (feature groups of FG = min(M, 64)); lane tile
// 2 token tiles x FG / 16 feature tiles, so each Kronecker operand built in registers feeds FG / 16
// matrix products. P^T blocks are loaded two blocks ahead into registers (two stages), then staged in
// LDS (double buffered).
// ---------------------------------------------------------------------------------------------
template <int M> constexpr int tmap_fg() { return M < 64 ? M : 64; }
template <int M> constexpr int tmap_fwd_threads() { return 64 * 4 * (M / tmap_fg<M>()); }

template <int D, int M>
struct TmapFwdSmem {
  alignas(16) bf16 xs[tm::TN][D + 8];
  alignas(16) bf16 pt[2][M][D + 8];   // P^T columns of the current / next block
};

// Four waves per SIMD (at most 128 VGPRs): the few bytes of spill this costs at D = 64, M = 128 are
// cheaper than the third wave's missing latency cover (measured).
// SYM: pt is a symmetrised table (atlas_tensor_map_symmetrize: P[a][b] + P[b][a] on b > a, zero on
// b < a), so the blocks of rows a >= D / 2 skip their products over the zero columns b < D / 2.
template <int D, int M, bool SYM>
__global__ __launch_bounds__(tmap_fwd_threads<M>()) __attribute__((amdgpu_waves_per_eu(4)))
void k_tmap_fwd(long n_tok, const bf16* __restrict__ x, const bf16* __restrict__ pt, bf16* __restrict__ out,
                int deg, bf16* __restrict__ pre) {
  constexpr int FG = tmap_fg<M>(), JT = FG / 16, NT = tmap_fwd_threads<M>(), K = D + D * D, NS = D / 32;
  constexpr int PV = M * D / 8;   // 16-byte vectors of one P^T block
  constexpr int PVT = (PV + NT - 1) / NT;
  __shared__ TmapFwdSmem<D, M> sm;
  const int tid = threadIdx.x, lane = lane_id(), w = threadIdx.x >> 6;
  const int g = lane >> 4, i = lane & 15;
  const int rg = w & 3, cg = w >> 2;     // tokens 32 rg .., features FG cg ..
  const long n0 = (long)blockIdx.x * tm::TN;
  const uint32_t xbytes = (uint32_t)(min((long)tm::TN, n_tok - n0) * D * 2);
  const rsrc_t rx = make_rsrc(x + n0 * D, xbytes);
  const rsrc_t rp = make_rsrc(pt, (uint32_t)(M * K * 2));

  // x tile -> LDS (rows past N read as zeros)
  for (int v = tid; v < tm::TN * D / 8; v += NT) {
    const int r = v / (D / 8), c8 = v % (D / 8);
    *reinterpret_cast<u32x4v*>(&sm.xs[r][c8 * 8]) = bld16(rx, (uint32_t)((r * D + c8 * 8) * 2));
  }
  // P^T block kb: columns kb*D .. of every feature row j (vector v: row v / (D/8), 8 columns)
  u32x4v pf0[PVT], pf1[PVT];
  // PACK (the symmetrised table at d = 64): the packed block order of tm::kPackQuad; otherwise block
  // kb is row kb - 1 of x x^T (kb 0: the linear rows). Blocks past the last read as zeros.
  constexpr bool PACK = SYM && D == 64 && NS == 2;
  constexpr int NBLK = PACK ? tm::kNPack : D + 1;
  auto p_load = [&](u32x4v (&pf)[PVT], int kb) {
#pragma unroll
    for (int u = 0; u < PVT; ++u) {
      const int v = tid + u * NT;
      const int j = v / (D / 8), c8 = v % (D / 8);
      int col = kb * D + c8 * 8;
      if constexpr (PACK) {
        if (kb >= tm::kPackQuad) {   // four 16-column pieces: rows a0 + (c8 >> 1), columns lo + 8 (c8 & 1)
          const int qv = kb - tm::kPackQuad, lo = qv < 4 ? 16 : 48, a0 = lo + 4 * (qv & 3);
          col = (a0 + (c8 >> 1) + 1) * D + lo + 8 * (c8 & 1);
        }
      }
      pf[u] = bld16(rp, (v < PV && kb < NBLK) ? (uint32_t)((j * K + col) * 2) : kOob);
    }
  };
  auto p_store = [&](const u32x4v (&pf)[PVT], int buf) {
#pragma unroll
    for (int u = 0; u < PVT; ++u) {
      const int v = tid + u * NT;
      if (v < PV) *reinterpret_cast<u32x4v*>(&sm.pt[buf][v / (D / 8)][(v % (D / 8)) * 8]) = pf[u];
    }
  };
  p_load(pf0, 0);
  p_store(pf0, 0);
  p_load(pf0, 1);
  p_load(pf1, 2);
  __syncthreads();

  // x_b of this lane's k slots, per token tile: b = 32 s + 8 g + e
  float xb[2][NS][8];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const bf16x8 v = *reinterpret_cast<const bf16x8*>(&sm.xs[32 * rg + 16 * nt + i][32 * s + 8 * g]);
#pragma unroll
      for (int e = 0; e < 8; ++e) xb[nt][s][e] = static_cast<float>(v[e]);
    }

  f32x4 acc[JT][2];
#pragma unroll
  for (int jt = 0; jt < JT; ++jt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) acc[jt][nt] = zero4();

  // block kb from LDS buffer kb & 1; register stage `pf` holds block kb + 1 and is refilled with
  // block kb + 3 after its store; the products start at column tile S0 (compile time)
  auto block = [&](int kb, u32x4v (&pf)[PVT], auto s0c) {
    constexpr int S0 = decltype(s0c)::value;
    const int buf = kb & 1;

    float xa[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)   // x_a of the block's row a = kb - 1 (unused in block 0)
      xa[nt] = static_cast<float>(sm.xs[32 * rg + 16 * nt + i][kb > 0 ? kb - 1 : 0]);
#pragma unroll
    for (int s = S0; s < NS; ++s) {
      bf16x8 fb[2];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        if (kb == 0) {   // workgroup-uniform: the linear block is x itself
          fb[nt] = frag_row(&sm.xs[0][0], D + 8, 32 * rg + 16 * nt, 32 * s);
        } else {         // x_a * x_b, rounded to bf16 like the materialised Kronecker features
#pragma unroll
          for (int e = 0; e < 8; ++e) fb[nt][e] = static_cast<bf16>(xa[nt] * xb[nt][s][e]);
        }
      }
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) {
        const bf16x8 fa = frag_row(&sm.pt[buf][0][0], D + 8, FG * cg + 16 * jt, 32 * s);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) acc[jt][nt] = mma_bf16(fa, fb[nt], acc[jt][nt]);
      }
    }
    if (kb + 1 < NBLK) {
      p_store(pf, buf ^ 1);
      p_load(pf, kb + 3);   // past the last block: out-of-range loads (zeros), never stored
    }
    __syncthreads();
  };
  // a quad of the packed order: four half-rows, two per k-step
  auto quad = [&](int kb, u32x4v (&pf)[PVT]) {
    const int buf = kb & 1;
    const int qv = kb - tm::kPackQuad, lo = qv < 4 ? 16 : 48, a0 = lo + 4 * (qv & 3);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      bf16x8 fb[2];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int tok = 32 * rg + 16 * nt + i;
        const float xa = static_cast<float>(sm.xs[tok][a0 + 2 * s + (g >> 1)]);
        const bf16x8 xv = *reinterpret_cast<const bf16x8*>(&sm.xs[tok][lo + 8 * (g & 1)]);
#pragma unroll
        for (int e = 0; e < 8; ++e) fb[nt][e] = static_cast<bf16>(xa * static_cast<float>(xv[e]));
      }
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) {
        const bf16x8 fa = frag_row(&sm.pt[buf][0][0], D + 8, FG * cg + 16 * jt, 32 * s);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) acc[jt][nt] = mma_bf16(fa, fb[nt], acc[jt][nt]);
      }
    }
    if (kb + 1 < NBLK) {
      p_store(pf, buf ^ 1);
      p_load(pf, kb + 3);
    }
    __syncthreads();
  };
  using all_t = std::integral_constant<int, 0>;
  using hi_t = std::integral_constant<int, NS / 2>;
  if constexpr (PACK) {
    // blocks 0 .. 16 over both k-steps, 17 .. 48 (rows 16 .. 47) over the upper one, then the quads;
    // even blocks take register stage pf0, odd ones pf1
    static_assert(tm::kPackQuad % 2 == 1 && (NBLK - tm::kPackQuad) % 2 == 0, "block parity");
    for (int kb = 0; kb < 16; kb += 2) {
      block(kb, pf0, all_t{});
      block(kb + 1, pf1, all_t{});
    }
    block(16, pf0, all_t{});
    for (int kb = 17; kb < tm::kPackQuad; kb += 2) {
      block(kb, pf1, hi_t{});
      block(kb + 1, pf0, hi_t{});
    }
    for (int kb = tm::kPackQuad; kb + 1 < NBLK; kb += 2) {
      quad(kb, pf1);
      quad(kb + 1, pf0);
    }
  } else {
  // blocks 0 .. KS - 1 over every column tile, then (SYM) the blocks of rows a >= D / 2 from tile
  // NS / 2 on; even blocks take register stage pf0, odd ones pf1
  constexpr int KS = (SYM && NS > 1) ? D / 2 + 1 : D + 1;
  static_assert(KS % 2 == 1 && D % 2 == 0, "block parity");
  for (int kb = 0; kb + 1 < KS; kb += 2) {
    block(kb, pf0, all_t{});
    block(kb + 1, pf1, all_t{});
  }
  block(KS - 1, pf0, all_t{});
  if constexpr (KS <= D) {
    block(KS, pf1, hi_t{});
    for (int kb = KS + 1; kb + 1 <= D; kb += 2) {
      block(kb, pf0, hi_t{});
      block(kb + 1, pf1, hi_t{});
    }
    block(D, pf0, hi_t{});
  }
  }

  // phi^T tiles: lane (g, i) holds phi[token 32 rg + 16 nt + i][feature FG cg + 16 jt + 4 g + r]
  const uint32_t obytes = (uint32_t)(min((long)tm::TN, n_tok - n0) * M * 2);
  const rsrc_t ro = make_rsrc(out + n0 * M, obytes);
  const rsrc_t rpre = make_rsrc(pre ? pre + n0 * M : out, pre ? obytes : 0u);
#pragma unroll
  for (int jt = 0; jt < JT; ++jt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int r = 32 * rg + 16 * nt + i, j = FG * cg + 16 * jt + 4 * g;
      const uint32_t off = (uint32_t)((r * M + j) * 2);
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = acc[jt][nt][e];
      if (deg > 1) {   // uniform
        u32x2v p;
        p[0] = pack_bf16x2(v[0], v[1]);
        p[1] = pack_bf16x2(v[2], v[3]);
        bst8(rpre, off, p);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = poly_map(v[e], deg);
      }
      u32x2v o;
      o[0] = pack_bf16x2(v[0], v[1]);
      o[1] = pack_bf16x2(v[2], v[3]);
      bst8(ro, off, o);
    }
}

// ---------------------------------------------------------------------------------------------
// backward: waves = 4 (token groups of 32) x D / 32 (feature halves of 32); lane tile 2 x 2
// ---------------------------------------------------------------------------------------------
template <int D, int M>
struct TmapBwdSmem {
  alignas(16) bf16 xs[tm::TN][D + 8];
  alignas(16) bf16 pb[2][D][M + 8];       // rows of P for the current / next block
  float t1[D / 32][tm::TN][D + 1];        // sum over b of G[n, a, b] x[n, b], per feature half of b
};

// SYM: proj is the symmetrised table (zero where b < a), so the blocks of rows a >= D / 2 only have
// products over b >= D / 2: there the two feature-half waves of a token group split its two token
// tiles instead of the feature halves (half the matrix-core work), the third term of a wave whose
// b half is the lower one is handed over through t1[0][n][b >= D / 2], which no block writes
// otherwise, and the second term lands whole in t1[1][n][a].
template <int D, int M, bool SYM = false>
__global__ __launch_bounds__(64 * 4 * (D / 32)) void k_tmap_bwd(long n_tok, const bf16* __restrict__ x,
                                                                   const bf16* __restrict__ proj,
                                                                   const bf16* __restrict__ dout,
                                                                   bf16* __restrict__ dx, int deg,
                                                                   const bf16* __restrict__ pre) {
  constexpr int NW = 4 * (D / 32), NT = 64 * NW, NK = M / 32;
  constexpr int PV = D * M / 8;   // 16-byte vectors of one block of D rows of P
  constexpr int PVT = (PV + NT - 1) / NT;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  TmapBwdSmem<D, M>& sm = *reinterpret_cast<TmapBwdSmem<D, M>*>(smem_raw);
  const int tid = threadIdx.x, lane = lane_id(), w = threadIdx.x >> 6;
  const int g = lane >> 4, i = lane & 15;
  const int rg = w & 3, cb = w >> 2;     // tokens 32 rg .., features (b, c) 32 cb ..
  const long n0 = (long)blockIdx.x * tm::TN;
  const long nrow = min((long)tm::TN, n_tok - n0);
  const rsrc_t rx = make_rsrc(x + n0 * D, (uint32_t)(nrow * D * 2));
  const rsrc_t rd = make_rsrc(dout + n0 * M, (uint32_t)(nrow * M * 2));
  const rsrc_t rp = make_rsrc(proj, (uint32_t)((D + D * D) * M * 2));

  for (int v = tid; v < tm::TN * D / 8; v += NT) {
    const int r = v / (D / 8), c8 = v % (D / 8);
    *reinterpret_cast<u32x4v*>(&sm.xs[r][c8 * 8]) = bld16(rx, (uint32_t)((r * D + c8 * 8) * 2));
  }
  // P rows kb*D .. kb*D + D - 1 (kb 0: the linear rows, kb a + 1: row a of x x^T), loaded two
  // blocks ahead into registers (two stages) and staged in LDS (double buffered)
  u32x4v pf0[PVT], pf1[PVT];
  auto p_load = [&](u32x4v (&pf)[PVT], int kb) {
#pragma unroll
    for (int u = 0; u < PVT; ++u) {
      const int v = tid + u * NT;
      const int r = v / (M / 8), c8 = v % (M / 8);
      pf[u] = bld16(rp, (v < PV && kb <= D) ? (uint32_t)(((kb * D + r) * M + c8 * 8) * 2) : kOob);
    }
  };
  auto p_store = [&](const u32x4v (&pf)[PVT], int buf) {
#pragma unroll
    for (int u = 0; u < PVT; ++u) {
      const int v = tid + u * NT;
      if (v < PV) *reinterpret_cast<u32x4v*>(&sm.pb[buf][v / (M / 8)][(v % (M / 8)) * 8]) = pf[u];
    }
  };
  // dphi of this lane's tokens as k operands over j (kept for the whole launch); with the
  // elementwise map, dphi = dout * map'(pre)
  const rsrc_t rpre = make_rsrc(pre ? pre + n0 * M : dout, pre ? (uint32_t)(nrow * M * 2) : 0u);
  bf16x8 fd[2][NK];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) {
      const uint32_t off = (uint32_t)(((32 * rg + 16 * nt + i) * M + 32 * ks + 8 * g) * 2);
      fd[nt][ks] = __builtin_bit_cast(bf16x8, bld16(rd, off));
      if (deg > 1) {   // uniform
        const bf16x8 pv = __builtin_bit_cast(bf16x8, bld16(rpre, off));
#pragma unroll
        for (int e = 0; e < 8; ++e)
          fd[nt][ks][e] = static_cast<bf16>(static_cast<float>(fd[nt][ks][e]) *
                                            poly_map_grad(static_cast<float>(pv[e]), deg));
      }
    }
  p_load(pf0, 0);
  p_store(pf0, 0);
  p_load(pf0, 1);
  p_load(pf1, 2);
  __syncthreads();

  // x[n, b] at this lane's tile positions: b = 32 cb + 16 bt + 4 g + r, n = 32 rg + 16 nt + i
  float xc[2][2][4];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
#pragma unroll
    for (int bt = 0; bt < 2; ++bt)
#pragma unroll
      for (int r = 0; r < 4; ++r) xc[nt][bt][r] = static_cast<float>(sm.xs[32 * rg + 16 * nt + i][32 * cb + 16 * bt + 4 * g + r]);

  f32x4 acc[2][2];   // [bt][nt]: dx^T tiles (linear term + third term)
#pragma unroll
  for (int bt = 0; bt < 2; ++bt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) acc[bt][nt] = zero4();

  // Software pipeline over the blocks of K: step kb forms G's tiles of block kb (matrix cores,
  // P block from LDS buffer kb & 1) while the vector units consume block kb - 1's tiles, which the
  // previous step left in the other register set; one barrier per block. Register stage `pf`
  // holds block kb + 1 and is refilled with kb + 3.
  auto mma = [&](int kb, f32x4 (&gt)[2][2]) {
    const int buf = kb & 1;
#pragma unroll
    for (int bt = 0; bt < 2; ++bt)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) gt[bt][nt] = zero4();
    // SYM at d = 64: rows a in [16, 32) are zero for b < 16, the first tile of the lower feature half
    if (SYM && D == 64 && cb == 0 && kb > D / 4 && kb <= D / 2) {   // wave-uniform
#pragma unroll
      for (int ks = 0; ks < NK; ++ks) {
        const bf16x8 fp1 = frag_row(&sm.pb[buf][0][0], M + 8, 16, 32 * ks);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) gt[1][nt] = mma_bf16(fp1, fd[nt][ks], gt[1][nt]);
      }
      return;
    }
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) {
      bf16x8 fp[2];
#pragma unroll
      for (int bt = 0; bt < 2; ++bt) fp[bt] = frag_row(&sm.pb[buf][0][0], M + 8, 32 * cb + 16 * bt, 32 * ks);
#pragma unroll
      for (int bt = 0; bt < 2; ++bt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) gt[bt][nt] = mma_bf16(fp[bt], fd[nt][ks], gt[bt][nt]);
    }
  };
  auto epi = [&](int kb, const f32x4 (&gt)[2][2]) {
    if (kb == 0) {   // workgroup-uniform: the linear rows give dx directly
#pragma unroll
      for (int bt = 0; bt < 2; ++bt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) acc[bt][nt] += gt[bt][nt];
    } else {
      const int a = kb - 1;
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int n = 32 * rg + 16 * nt + i;
        const float xa = static_cast<float>(sm.xs[n][a]);
        float part = 0.f;
#pragma unroll
        for (int bt = 0; bt < 2; ++bt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            acc[bt][nt][r] += gt[bt][nt][r] * xa;          // G[n, a, c] x[n, a] for c = b
            part += gt[bt][nt][r] * xc[nt][bt][r];         // G[n, a, b] x[n, b]
          }
        part = xsum_rows(part);                             // over the four lane rows (all 32 b)
        if (g == 0) sm.t1[cb][n][a] = part;
      }
    }
  };
  auto step = [&](int kb, u32x4v (&pf)[PVT], f32x4 (&gcur)[2][2], const f32x4 (&gprev)[2][2]) {
    mma(kb, gcur);
    if (kb > 0) epi(kb - 1, gprev);
    if (kb < D) {
      p_store(pf, (kb & 1) ^ 1);   // buffer of block kb - 1, whose reads ended before the last barrier
      p_load(pf, kb + 3);          // past the last block: out-of-range loads (zeros), never stored
    }
    __syncthreads();
  };
  f32x4 gA[2][2], gB[2][2];
  if constexpr (!SYM || D != 64) {
    for (int kb = 0; kb <= D; kb += 2) {
      step(kb, pf0, gA, gB);
      if (kb + 1 <= D) step(kb + 1, pf1, gB, gA);
    }
    epi(D, gA);   // D is even: the last block's tiles are in gA
  } else {
    // blocks 0 .. D / 2 (the linear rows and a < D / 2) as above
    for (int kb = 0; kb < D / 2; kb += 2) {
      step(kb, pf0, gA, gB);
      step(kb + 1, pf1, gB, gA);
    }
    step(D / 2, pf0, gA, gB);
    // blocks a + 1 with a >= D / 2: tiles b = D / 2 + 16 bt, tokens 32 rg + 16 cb (token tile nt = cb)
    bf16x8 fdh[NK];
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) fdh[ks] = cb ? fd[1][ks] : fd[0][ks];
    const int nh = 32 * rg + 16 * cb + i;
    float xh[2][4];
    f32x4 accH[2];
#pragma unroll
    for (int bt = 0; bt < 2; ++bt) {
      accH[bt] = zero4();
#pragma unroll
      for (int r = 0; r < 4; ++r) xh[bt][r] = static_cast<float>(sm.xs[nh][D / 2 + 16 * bt + 4 * g + r]);
    }
    auto mma_h = [&](int kb, f32x4 (&gt)[2]) {
      const int buf = kb & 1;
#pragma unroll
      for (int bt = 0; bt < 2; ++bt) gt[bt] = zero4();
      if (kb > 3 * D / 4) {   // rows a >= 48: zero for b < 48, the first tile of the upper half
#pragma unroll
        for (int ks = 0; ks < NK; ++ks)
          gt[1] = mma_bf16(frag_row(&sm.pb[buf][0][0], M + 8, D / 2 + 16, 32 * ks), fdh[ks], gt[1]);
        return;
      }
#pragma unroll
      for (int ks = 0; ks < NK; ++ks) {
#pragma unroll
        for (int bt = 0; bt < 2; ++bt)
          gt[bt] = mma_bf16(frag_row(&sm.pb[buf][0][0], M + 8, D / 2 + 16 * bt, 32 * ks), fdh[ks], gt[bt]);
      }
    };
    auto epi_h = [&](int kb, const f32x4 (&gt)[2]) {
      const int a = kb - 1;
      const float xa = static_cast<float>(sm.xs[nh][a]);
      float part = 0.f;
#pragma unroll
      for (int bt = 0; bt < 2; ++bt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          accH[bt][r] += gt[bt][r] * xa;
          part += gt[bt][r] * xh[bt][r];
        }
      part = xsum_rows(part);
      if (g == 0) sm.t1[1][nh][a] = part;
    };
    auto step_h = [&](int kb, u32x4v (&pf)[PVT], f32x4 (&gcur)[2], const f32x4 (&gprev)[2]) {
      mma_h(kb, gcur);
      epi_h(kb - 1, gprev);
      if (kb < D) {
        p_store(pf, (kb & 1) ^ 1);
        p_load(pf, kb + 3);
      }
      __syncthreads();
    };
    f32x4 hA[2], hB[2];
    mma_h(D / 2 + 1, hA);   // block D / 2 + 1, with the epilogue of block D / 2 (full tiles)
    epi(D / 2, gA);
    p_store(pf1, ((D / 2 + 1) & 1) ^ 1);
    p_load(pf1, D / 2 + 4);
    __syncthreads();
    for (int kb = D / 2 + 2; kb <= D; kb += 2) {
      step_h(kb, pf0, hB, hA);
      if (kb + 1 <= D) step_h(kb + 1, pf1, hA, hB);
    }
    epi_h(D, hB);   // D is even: the last block's tiles are in hB
    // the third term of the upper feature half: a wave of the upper half keeps its own token tile's,
    // a wave of the lower half hands its tile's over (t1[0][n][c >= D / 2] holds only this)
#pragma unroll
    for (int bt = 0; bt < 2; ++bt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int cc = D / 2 + 16 * bt + 4 * g + r;
        if (cb) {
          acc[bt][1][r] += accH[bt][r];
          sm.t1[0][nh][cc] = 0.f;
        } else {
          sm.t1[0][nh][cc] = accH[bt][r];
        }
      }
  }
  __syncthreads();   // t1 written by the other feature half's waves

  // dx[n, c] = acc (c = 32 cb + 16 bt + 4 g + r) + sum over the halves of t1[., n, c]
  const rsrc_t ro = make_rsrc(dx + n0 * D, (uint32_t)(nrow * D * 2));
#pragma unroll
  for (int bt = 0; bt < 2; ++bt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int n = 32 * rg + 16 * nt + i, c = 32 * cb + 16 * bt + 4 * g;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float s = acc[bt][nt][r];
#pragma unroll
        for (int h = 0; h < D / 32; ++h) s += sm.t1[h][n][c + r];
        v[r] = s;
      }
      u32x2v o;
      o[0] = pack_bf16x2(v[0], v[1]);
      o[1] = pack_bf16x2(v[2], v[3]);
      bst8(ro, (uint32_t)((n * D + c) * 2), o);
    }
}

template <int D, int M, bool SYM = false>
hipError_t launch_tmap_fwd(long n, const bf16* x, const bf16* pt, bf16* out, int deg, bf16* pre, hipStream_t s) {
  const unsigned grid = (unsigned)((n + tm::TN - 1) / tm::TN);
  hipLaunchKernelGGL((k_tmap_fwd<D, M, SYM>), dim3(grid), dim3(tmap_fwd_threads<M>()), 0, s, n, x, pt, out, deg, pre);
  return hipGetLastError();
}

// The symmetrised projection (both layouts): x x^T is symmetric, so its projection keeps only
// a <= b: ps[D + a D + b] = P[D + a D + b] + P[D + b D + a] (b > a), P[D + a D + a] (b = a), 0 (b < a);
// the linear rows are copied. ps [K][M] (the backward's layout) and pst [M][K] (the forward's).
template <typename T>
__global__ __launch_bounds__(256) void k_tmap_symmetrize(int D, int M, const T* __restrict__ p, T* __restrict__ ps,
                                                         T* __restrict__ pst) {
  const int K = D + D * D;
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)K * M) return;
  const int r = (int)(idx / M), j = (int)(idx % M);
  float v;
  if (r < D) {
    v = static_cast<float>(p[idx]);
  } else {
    const int a = (r - D) / D, b = (r - D) % D;
    v = b < a ? 0.f : static_cast<float>(p[idx]);
    if (b > a) v += static_cast<float>(p[(long)(D + b * D + a) * M + j]);
  }
  ps[idx] = static_cast<T>(v);
  pst[(long)j * K + r] = static_cast<T>(v);
}

template <int D, int M, bool SYM = false>
hipError_t launch_tmap_bwd(long n, const bf16* x, const bf16* p, const bf16* dout, bf16* dx, int deg, const bf16* pre,
                           hipStream_t s) {
  const size_t smem = sizeof(TmapBwdSmem<D, M>);
  hipError_t err = set_dyn_smem(reinterpret_cast<const void*>(&k_tmap_bwd<D, M, SYM>), smem);
  if (err != hipSuccess) return err;
  const unsigned grid = (unsigned)((n + tm::TN - 1) / tm::TN);
  hipLaunchKernelGGL((k_tmap_bwd<D, M, SYM>), dim3(grid), dim3(64 * 4 * (D / 32)), smem, s, n, x, p, dout, dx, deg,
                     pre);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// General kernels: fp32 inputs (fp32 operands on v_mfma_f32_16x16x4f32, fp32 accumulate: the
// map in x.dtype as the reference runs it) and bf16 inputs at the sizes the kernels above are not
// built for. d_in in {16, 32, 64}, d_out a multiple of 16 up to 128. One workgroup (4 waves) per 64
// tokens, wave w owning tokens 16 w .. 16 w + 15; P's blocks of d_in rows (block 0 the linear
// rows, block a + 1 the rows that multiply x_a x) are staged in LDS as fp32 pb[b][o], one block at
// a time, with the next block prefetched into registers while the current one is consumed.
//   forward   phi[n, o] = sum_blk sum_b A_blk[n, b] pb_blk[b, o],  A_0 = x,  A_{a+1} = x_a x
//   backward  G_blk[n, b] = sum_o dphi[n, o] pb_blk[b, o]; dx[n, b] += G_0[n, b] + x[n, a] G_{a+1}[n, b]
//             and dx[n, a] += sum_b G_{a+1}[n, b] x[n, b] (a 16-lane sum, collected in an LDS table)
// ---------------------------------------------------------------------------------------------
namespace tg {
constexpr int TN = 64;      // tokens per workgroup
constexpr int NT = 256;     // threads
constexpr int MMAX = 128;   // largest d_out
}

// Four consecutive elements as fp32 (8-byte aligned bf16 or 16-byte aligned fp32).
__device__ __forceinline__ float4 ld4f(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 ld4f(const bf16* p) {
  const uint2 u = *reinterpret_cast<const uint2*>(p);
  return make_float4(__builtin_bit_cast(float, u.x << 16), __builtin_bit_cast(float, u.x & 0xffff0000u),
                     __builtin_bit_cast(float, u.y << 16), __builtin_bit_cast(float, u.y & 0xffff0000u));
}

template <int D, int PITCH>
struct TgSmem {
  float xs[tg::TN][D + 1];                // x of the workgroup's tokens (zero past n_tok)
  alignas(16) float pb[D][PITCH];         // the current P block, pb[b][o]
  float t1[tg::TN][D + 1];   // backward: the row term sum_b G_{a+1}[n, b] x[n, b] at [n][a]
};

// x rows n0 .. n0 + 63 into xs (fp32, zeros past n_tok)
template <typename T, int D, int PITCH>
__device__ __forceinline__ void tg_load_x(TgSmem<D, PITCH>& sm, const T* x, long n0, long n_tok) {
  for (int u = threadIdx.x; u < tg::TN * D / 4; u += tg::NT) {
    const int r = u / (D / 4), c = (u % (D / 4)) * 4;
    const float4 v = n0 + r < n_tok ? ld4f(x + (n0 + r) * D + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    sm.xs[r][c] = v.x; sm.xs[r][c + 1] = v.y; sm.xs[r][c + 2] = v.z; sm.xs[r][c + 3] = v.w;
  }
}

template <typename T, int D>
__global__ __launch_bounds__(tg::NT) void k_tmap_gen_fwd(long n_tok, int M, const T* __restrict__ x,
                                                         const T* __restrict__ pt, T* __restrict__ out, int deg,
                                                         T* __restrict__ pre) {
  constexpr int KK = D / 4, K = D + D * D;
  constexpr int VPT = tg::MMAX * D / 4 / tg::NT;   // P^T vectors per thread and block (at M = 128)
  __shared__ TgSmem<D, tg::MMAX + 16> sm;          // pitch: 4 k rows x 16 columns hit 64 banks
  const int tid = threadIdx.x, l = lane_id(), w = wave_id();
  const int row = l & 15, kq = l >> 4;
  const long n0 = (long)blockIdx.x * tg::TN;
  const int JT = M / 16, nvec = M * D / 4;
  tg_load_x<T, D>(sm, x, n0, n_tok);
  // P block blk from P^T [M][K]: pb[b][o] = P^T[o][blk D + b], four b per vector
  float4 pf[VPT];
  auto pload = [&](int blk) {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int v = tid + i * tg::NT;
      if (v < nvec) pf[i] = ld4f(pt + (size_t)(v / KK) * K + blk * D + (v % KK) * 4);
    }
  };
  auto pstore = [&]() {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int v = tid + i * tg::NT;
      if (v < nvec) {
        const int o = v / KK, b = (v % KK) * 4;
        sm.pb[b][o] = pf[i].x; sm.pb[b + 1][o] = pf[i].y; sm.pb[b + 2][o] = pf[i].z; sm.pb[b + 3][o] = pf[i].w;
      }
    }
  };
  pload(0);
  __syncthreads();
  float xv[KK];   // x[n][4 kk + kq] of this lane's token row
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) xv[kk] = sm.xs[16 * w + row][4 * kk + kq];
  f32x4 acc[tg::MMAX / 16];
#pragma unroll
  for (int j = 0; j < tg::MMAX / 16; ++j) acc[j] = zero4();
  for (int blk = 0; blk <= D; ++blk) {
    __syncthreads();   // every wave is done with the previous block
    pstore();
    __syncthreads();
    if (blk < D) pload(blk + 1);
    const float xa = blk == 0 ? 1.f : sm.xs[16 * w + row][blk - 1];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const float av = xa * xv[kk];
#pragma unroll
      for (int j = 0; j < tg::MMAX / 16; ++j)
        if (j < JT) acc[j] = MM<float>::mma(av, sm.pb[4 * kk + kq][16 * j + row], acc[j]);
    }
  }
  // acc[j][r] = phi[token 16 w + 4 kq + r][feature 16 j + row]
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const long n = n0 + 16 * w + 4 * kq + r;
    if (n >= n_tok) continue;
#pragma unroll
    for (int j = 0; j < tg::MMAX / 16; ++j) {
      if (j >= JT) continue;
      const size_t o = (size_t)n * M + 16 * j + row;
      const float v = acc[j][r];
      if (deg > 1) {
        pre[o] = from_f32<T>(v);
        out[o] = from_f32<T>(poly_map(v, deg));
      } else {
        out[o] = from_f32<T>(v);
      }
    }
  }
}

template <typename T, int D>
__global__ __launch_bounds__(tg::NT) void k_tmap_gen_bwd(long n_tok, int M, const T* __restrict__ x,
                                                         const T* __restrict__ p, const T* __restrict__ dout,
                                                         T* __restrict__ dx, int deg, const T* __restrict__ pre) {
  constexpr int JD = D / 16, KO = tg::MMAX / 4;
  constexpr int VPT = tg::MMAX * D / 4 / tg::NT;
  __shared__ TgSmem<D, tg::MMAX + 4> sm;   // pitch: 16 rows x 4 k columns hit 64 banks
  const int tid = threadIdx.x, l = lane_id(), w = wave_id();
  const int row = l & 15, kq = l >> 4;
  const long n0 = (long)blockIdx.x * tg::TN;
  const int MQ = M / 4, nvec = M * D / 4;
  tg_load_x<T, D>(sm, x, n0, n_tok);
  for (int u = tid; u < tg::TN * (D + 1); u += tg::NT) (&sm.t1[0][0])[u] = 0.f;
  // P block blk from P [K][M]: pb[b][o] = P[blk D + b][o], four o per vector
  float4 pf[VPT];
  auto pload = [&](int blk) {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int v = tid + i * tg::NT;
      if (v < nvec) pf[i] = ld4f(p + (size_t)(blk * D + v / MQ) * M + (v % MQ) * 4);
    }
  };
  auto pstore = [&]() {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int v = tid + i * tg::NT;
      if (v < nvec) *reinterpret_cast<float4*>(&sm.pb[v / MQ][(v % MQ) * 4]) = pf[i];
    }
  };
  pload(0);
  // dphi (scaled by the map's derivative at pre) of this lane's token row, k = 4 kk + kq
  float dp[KO];
  {
    const long n = n0 + 16 * w + row;
#pragma unroll
    for (int kk = 0; kk < KO; ++kk) {
      float v = 0.f;
      if (kk < MQ && n < n_tok) {
        const size_t o = (size_t)n * M + 4 * kk + kq;
        v = to_f32(dout[o]);
        if (deg > 1) v *= poly_map_grad(to_f32(pre[o]), deg);
      }
      dp[kk] = v;
    }
  }
  __syncthreads();
  float xc[JD][4], dxc[JD][4];   // x and dx at [token 16 w + 4 kq + r][16 jd + row]
#pragma unroll
  for (int jd = 0; jd < JD; ++jd)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      xc[jd][r] = sm.xs[16 * w + 4 * kq + r][16 * jd + row];
      dxc[jd][r] = 0.f;
    }
  for (int blk = 0; blk <= D; ++blk) {
    __syncthreads();
    pstore();
    __syncthreads();
    if (blk < D) pload(blk + 1);
    f32x4 G[JD];
#pragma unroll
    for (int jd = 0; jd < JD; ++jd) G[jd] = zero4();
#pragma unroll
    for (int kk = 0; kk < KO; ++kk) {
      if (kk >= MQ) break;
#pragma unroll
      for (int jd = 0; jd < JD; ++jd) G[jd] = MM<float>::mma(dp[kk], sm.pb[16 * jd + row][4 * kk + kq], G[jd]);
    }
    // G[jd][r] = G_blk[token 16 w + 4 kq + r][b = 16 jd + row]
    if (blk == 0) {
#pragma unroll
      for (int jd = 0; jd < JD; ++jd)
#pragma unroll
        for (int r = 0; r < 4; ++r) dxc[jd][r] += G[jd][r];
    } else {
      const int a = blk - 1;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float xa = sm.xs[16 * w + 4 * kq + r][a];
        float rs = 0.f;
#pragma unroll
        for (int jd = 0; jd < JD; ++jd) {
          dxc[jd][r] += xa * G[jd][r];
          rs += G[jd][r] * xc[jd][r];
        }
        rs = row_sum16(rs);
        if (row == 0) sm.t1[16 * w + 4 * kq + r][a] = rs;   // rows of this wave only
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const long n = n0 + 16 * w + 4 * kq + r;
    if (n >= n_tok) continue;
#pragma unroll
    for (int jd = 0; jd < JD; ++jd) {
      const int c = 16 * jd + row;
      dx[(size_t)n * D + c] = from_f32<T>(dxc[jd][r] + sm.t1[16 * w + 4 * kq + r][c]);
    }
  }
}

template <typename T>
hipError_t tmap_gen_fwd(int d, int m, long n, const T* x, const T* pt, T* out, int deg, T* pre, hipStream_t s) {
  const dim3 grid((unsigned)((n + tg::TN - 1) / tg::TN)), block(tg::NT);
  if (d == 16) hipLaunchKernelGGL((k_tmap_gen_fwd<T, 16>), grid, block, 0, s, n, m, x, pt, out, deg, pre);
  else if (d == 32) hipLaunchKernelGGL((k_tmap_gen_fwd<T, 32>), grid, block, 0, s, n, m, x, pt, out, deg, pre);
  else if (d == 64) hipLaunchKernelGGL((k_tmap_gen_fwd<T, 64>), grid, block, 0, s, n, m, x, pt, out, deg, pre);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}
template <typename T>
hipError_t tmap_gen_bwd(int d, int m, long n, const T* x, const T* p, const T* dout, T* dx, int deg, const T* pre,
                        hipStream_t s) {
  const dim3 grid((unsigned)((n + tg::TN - 1) / tg::TN)), block(tg::NT);
  if (d == 16) hipLaunchKernelGGL((k_tmap_gen_bwd<T, 16>), grid, block, 0, s, n, m, x, p, dout, dx, deg, pre);
  else if (d == 32) hipLaunchKernelGGL((k_tmap_gen_bwd<T, 32>), grid, block, 0, s, n, m, x, p, dout, dx, deg, pre);
  else if (d == 64) hipLaunchKernelGGL((k_tmap_gen_bwd<T, 64>), grid, block, 0, s, n, m, x, p, dout, dx, deg, pre);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

bool tmap_fast(int d, int m) { return (d == 32 || d == 64) && (m == 32 || m == 64 || m == 128); }

// bf16: d_in in {32, 64}, d_out in {32, 64, 128} on the kernels above, other sizes on the general ones
hipError_t tmap_fwd(int d, int m, long n, const bf16* x, const bf16* pt, bf16* out, int deg, bf16* pre, hipStream_t s) {
  if (!tmap_fast(d, m)) return tmap_gen_fwd<bf16>(d, m, n, x, pt, out, deg, pre, s);
  if (d == 64 && m == 128) return launch_tmap_fwd<64, 128>(n, x, pt, out, deg, pre, s);
  if (d == 64 && m == 64) return launch_tmap_fwd<64, 64>(n, x, pt, out, deg, pre, s);
  if (d == 64 && m == 32) return launch_tmap_fwd<64, 32>(n, x, pt, out, deg, pre, s);
  if (d == 32 && m == 128) return launch_tmap_fwd<32, 128>(n, x, pt, out, deg, pre, s);
  if (d == 32 && m == 64) return launch_tmap_fwd<32, 64>(n, x, pt, out, deg, pre, s);
  if (d == 32 && m == 32) return launch_tmap_fwd<32, 32>(n, x, pt, out, deg, pre, s);
  return hipErrorInvalidValue;
}
// The same with a symmetrised table: the d_in = 64 kernels skip its zero lower triangle.
hipError_t tmap_fwd_sym(int d, int m, long n, const bf16* x, const bf16* pt, bf16* out, int deg, bf16* pre,
                        hipStream_t s) {
  if (d == 64 && m == 128) return launch_tmap_fwd<64, 128, true>(n, x, pt, out, deg, pre, s);
  if (d == 64 && m == 64) return launch_tmap_fwd<64, 64, true>(n, x, pt, out, deg, pre, s);
  if (d == 64 && m == 32) return launch_tmap_fwd<64, 32, true>(n, x, pt, out, deg, pre, s);
  return tmap_fwd(d, m, n, x, pt, out, deg, pre, s);
}
hipError_t tmap_bwd(int d, int m, long n, const bf16* x, const bf16* p, const bf16* dout, bf16* dx, int deg,
                    const bf16* pre, hipStream_t s) {
  if (!tmap_fast(d, m)) return tmap_gen_bwd<bf16>(d, m, n, x, p, dout, dx, deg, pre, s);
  if (d == 64 && m == 128) return launch_tmap_bwd<64, 128>(n, x, p, dout, dx, deg, pre, s);
  if (d == 64 && m == 64) return launch_tmap_bwd<64, 64>(n, x, p, dout, dx, deg, pre, s);
  if (d == 64 && m == 32) return launch_tmap_bwd<64, 32>(n, x, p, dout, dx, deg, pre, s);
  if (d == 32 && m == 128) return launch_tmap_bwd<32, 128>(n, x, p, dout, dx, deg, pre, s);
  if (d == 32 && m == 64) return launch_tmap_bwd<32, 64>(n, x, p, dout, dx, deg, pre, s);
  if (d == 32 && m == 32) return launch_tmap_bwd<32, 32>(n, x, p, dout, dx, deg, pre, s);
  return hipErrorInvalidValue;
}
// The same with a symmetrised table: the d_in = 64 kernels skip its zero lower triangle.
hipError_t tmap_bwd_sym(int d, int m, long n, const bf16* x, const bf16* ps, const bf16* dout, bf16* dx, int deg,
                        const bf16* pre, hipStream_t s) {
  if (d == 64 && m == 128) return launch_tmap_bwd<64, 128, true>(n, x, ps, dout, dx, deg, pre, s);
  if (d == 64 && m == 64) return launch_tmap_bwd<64, 64, true>(n, x, ps, dout, dx, deg, pre, s);
  if (d == 64 && m == 32) return launch_tmap_bwd<64, 32, true>(n, x, ps, dout, dx, deg, pre, s);
  return tmap_bwd(d, m, n, x, ps, dout, dx, deg, pre, s);
}

}  // namespace atlas

// ---------------------------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------------------------
#include "../../include/atlas_mem.h"

namespace {
bool tmap_dims_ok(int64_t n, int d_in, int d_out) {
  return n >= 0 && n < ((int64_t)1 << 40) && (d_in == 16 || d_in == 32 || d_in == 64) && d_out >= 16 &&
         d_out <= 128 && d_out % 16 == 0;
}
bool tmap_misaligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) != 0; }
}  // namespace

extern "C" {

int atlas_tensor_map_fwd(int dtype, int64_t n, int d_in, int d_out, int degree, const void* x, const void* proj_t,
                         void* out, void* pre, void* stream) {
  if (dtype != ATLAS_DT_BF16 && dtype != ATLAS_DT_F32) return ATLAS_MEM_ERR_DTYPE;
  if (!tmap_dims_ok(n, d_in, d_out) || degree < 1 || degree > 16) return ATLAS_MEM_ERR_SHAPE;
  if (!x || !proj_t || !out || (degree > 1 && !pre)) return ATLAS_MEM_ERR_NULL;
  if (tmap_misaligned(x) || tmap_misaligned(proj_t) || tmap_misaligned(out) || tmap_misaligned(pre))
    return ATLAS_MEM_ERR_ALIGN;
  if (n == 0) return ATLAS_MEM_OK;
  if (dtype == ATLAS_DT_F32) {
    const hipError_t err = atlas::tmap_gen_fwd<float>(d_in, d_out, (long)n, static_cast<const float*>(x),
                                                      static_cast<const float*>(proj_t), static_cast<float*>(out),
                                                      degree, degree > 1 ? static_cast<float*>(pre) : nullptr,
                                                      static_cast<hipStream_t>(stream));
    return err == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
  }
  const hipError_t err = atlas::tmap_fwd(d_in, d_out, (long)n, static_cast<const atlas::bf16*>(x),
                                         static_cast<const atlas::bf16*>(proj_t), static_cast<atlas::bf16*>(out),
                                         degree, degree > 1 ? static_cast<atlas::bf16*>(pre) : nullptr,
                                         static_cast<hipStream_t>(stream));
  return err == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

int atlas_tensor_map_symmetrize(int dtype, int d_in, int d_out, const void* proj, void* proj_sym, void* proj_sym_t,
                                void* stream) {
  if (dtype != ATLAS_DT_BF16 && dtype != ATLAS_DT_F32) return ATLAS_MEM_ERR_DTYPE;
  if (!tmap_dims_ok(0, d_in, d_out)) return ATLAS_MEM_ERR_SHAPE;
  if (!proj || !proj_sym || !proj_sym_t) return ATLAS_MEM_ERR_NULL;
  if (tmap_misaligned(proj) || tmap_misaligned(proj_sym) || tmap_misaligned(proj_sym_t)) return ATLAS_MEM_ERR_ALIGN;
  const long total = (long)(d_in + d_in * d_in) * d_out;
  const unsigned grid = (unsigned)((total + 255) / 256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == ATLAS_DT_F32)
    hipLaunchKernelGGL(atlas::k_tmap_symmetrize<float>, dim3(grid), dim3(256), 0, s, d_in, d_out,
                       static_cast<const float*>(proj), static_cast<float*>(proj_sym), static_cast<float*>(proj_sym_t));
  else
    hipLaunchKernelGGL(atlas::k_tmap_symmetrize<atlas::bf16>, dim3(grid), dim3(256), 0, s, d_in, d_out,
                       static_cast<const atlas::bf16*>(proj), static_cast<atlas::bf16*>(proj_sym),
                       static_cast<atlas::bf16*>(proj_sym_t));
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

int atlas_tensor_map_fwd_sym(int dtype, int64_t n, int d_in, int d_out, int degree, const void* x,
                             const void* proj_sym_t, void* out, void* pre, void* stream) {
  if (dtype != ATLAS_DT_BF16) return atlas_tensor_map_fwd(dtype, n, d_in, d_out, degree, x, proj_sym_t, out, pre, stream);
  if (!tmap_dims_ok(n, d_in, d_out) || degree < 1 || degree > 16) return ATLAS_MEM_ERR_SHAPE;
  if (!x || !proj_sym_t || !out || (degree > 1 && !pre)) return ATLAS_MEM_ERR_NULL;
  if (tmap_misaligned(x) || tmap_misaligned(proj_sym_t) || tmap_misaligned(out) || tmap_misaligned(pre))
    return ATLAS_MEM_ERR_ALIGN;
  if (n == 0) return ATLAS_MEM_OK;
  const hipError_t err = atlas::tmap_fwd_sym(d_in, d_out, (long)n, static_cast<const atlas::bf16*>(x),
                                             static_cast<const atlas::bf16*>(proj_sym_t), static_cast<atlas::bf16*>(out),
                                             degree, degree > 1 ? static_cast<atlas::bf16*>(pre) : nullptr,
                                             static_cast<hipStream_t>(stream));
  return err == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

int atlas_tensor_map_bwd(int dtype, int64_t n, int d_in, int d_out, int degree, const void* x, const void* proj,
                         const void* pre, const void* dout, void* dx, void* stream) {
  if (dtype != ATLAS_DT_BF16 && dtype != ATLAS_DT_F32) return ATLAS_MEM_ERR_DTYPE;
  if (!tmap_dims_ok(n, d_in, d_out) || degree < 1 || degree > 16) return ATLAS_MEM_ERR_SHAPE;
  if (!x || !proj || !dout || !dx || (degree > 1 && !pre)) return ATLAS_MEM_ERR_NULL;
  if (tmap_misaligned(x) || tmap_misaligned(proj) || tmap_misaligned(dout) || tmap_misaligned(dx) ||
      tmap_misaligned(pre))
    return ATLAS_MEM_ERR_ALIGN;
  if (n == 0) return ATLAS_MEM_OK;
  if (dtype == ATLAS_DT_F32) {
    const hipError_t err = atlas::tmap_gen_bwd<float>(d_in, d_out, (long)n, static_cast<const float*>(x),
                                                      static_cast<const float*>(proj), static_cast<const float*>(dout),
                                                      static_cast<float*>(dx), degree,
                                                      degree > 1 ? static_cast<const float*>(pre) : nullptr,
                                                      static_cast<hipStream_t>(stream));
    return err == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
  }
  const hipError_t err = atlas::tmap_bwd(d_in, d_out, (long)n, static_cast<const atlas::bf16*>(x),
                                         static_cast<const atlas::bf16*>(proj), static_cast<const atlas::bf16*>(dout),
                                         static_cast<atlas::bf16*>(dx), degree,
                                         degree > 1 ? static_cast<const atlas::bf16*>(pre) : nullptr,
                                         static_cast<hipStream_t>(stream));
  return err == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

int atlas_tensor_map_bwd_sym(int dtype, int64_t n, int d_in, int d_out, int degree, const void* x,
                             const void* proj_sym, const void* pre, const void* dout, void* dx, void* stream) {
  if (dtype != ATLAS_DT_BF16)
    return atlas_tensor_map_bwd(dtype, n, d_in, d_out, degree, x, proj_sym, pre, dout, dx, stream);
  if (!tmap_dims_ok(n, d_in, d_out) || degree < 1 || degree > 16) return ATLAS_MEM_ERR_SHAPE;
  if (!x || !proj_sym || !dout || !dx || (degree > 1 && !pre)) return ATLAS_MEM_ERR_NULL;
  if (tmap_misaligned(x) || tmap_misaligned(proj_sym) || tmap_misaligned(dout) || tmap_misaligned(dx) ||
      tmap_misaligned(pre))
    return ATLAS_MEM_ERR_ALIGN;
  if (n == 0) return ATLAS_MEM_OK;
  const hipError_t err = atlas::tmap_bwd_sym(d_in, d_out, (long)n, static_cast<const atlas::bf16*>(x),
                                             static_cast<const atlas::bf16*>(proj_sym),
                                             static_cast<const atlas::bf16*>(dout), static_cast<atlas::bf16*>(dx),
                                             degree, degree > 1 ? static_cast<const atlas::bf16*>(pre) : nullptr,
                                             static_cast<hipStream_t>(stream));
  return err == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

}  // extern "C"
