// gemm.hip - the cell's linear layers as batched bf16 matrix-core products: up to four independent
// problems per launch (the q / k / v / gate projections of the prologue share one launch, and so do
// their input gradients), fp32 accumulation, bf16 out. Replaces the forward and input-gradient
// products autograd forms for LinearNoBias to_q / to_k / to_v / to_out and the gate heads'
// Linear(dim, heads) (rnn_memory.py:486-489, :503-520); their weight gradients are wgrad.hip.
//
//   layout NT:  C[m, n] = sum_k A[m, k] Bt[n, k]    (y = x W^T: A = x [M, K], Bt = W [N, K])
//   layout NN:  C[m, n] = sum_k A[m, k] B[k, n]     (dx = dy W: A = dy [M, K], B = W [K, N])
//
// Workgroup tile 128 (m) x 128 (n), four waves of 64 x 64, K steps of 64 staged in LDS (double
// buffered, the next step's loads in registers). The matrix cores compute C^T tiles (Bt rows as the
// first operand), so each lane holds four consecutive n of one m and stores 8 bytes. Bt and A tiles
// are read as 16-byte row fragments; the NN layout's B tile is staged as stored ([k][n]) and read
// transposed (ds_read_b64_tr_b16). Rows past M / N / K read zeros through the buffer range check,
// columns past K or N through a per-thread mask.
#include "../../include/atlas_mem.h"
#include "mem_common.h"
#include "walk_common.h"

namespace atlas {

namespace gm {
constexpr int TM = 128, TN = 128, KS = 64;
constexpr int PA = KS + 8;        // pitch of the [row][k] tiles (A, and Bt for NT)
constexpr int PB = TN + 16;       // pitch of the NN layout's [k][n] tile (transposing reads)
constexpr int NT = 256;
constexpr int MAXP = 4;
struct Batch {
  const bf16* a[MAXP];
  const bf16* b[MAXP];
  bf16* c[MAXP];
  int n[MAXP];
  int k[MAXP];
};
template <bool NN>
struct Smem {
  alignas(16) bf16 a[2][TM][PA];
  alignas(16) bf16 b[2][NN ? KS : TN][NN ? PB : PA];
};
}  // namespace gm

template <bool NN>
__global__ __launch_bounds__(gm::NT) void k_gemm(long M, gm::Batch p) {
  using namespace gm;
  __shared__ Smem<NN> sm;
  const int z = blockIdx.z;
  const int N = p.n[z], K = p.k[z];
  const int n0 = TN * blockIdx.y;
  if (n0 >= N) return;   // workgroup-uniform, before any barrier
  const long m0 = (long)TM * blockIdx.x;
  const int tid = threadIdx.x, lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = w & 1, wn = w >> 1;
  const long mrows = min((long)TM, M - m0);
  const rsrc_t ra = make_rsrc(p.a[z] + m0 * K, (uint32_t)(mrows * K * 2));
  const rsrc_t rb = NN ? make_rsrc(p.b[z] + n0, (uint32_t)(((long)(K - 1) * N + (N - n0)) * 2))
                       : make_rsrc(p.b[z] + (long)n0 * K, (uint32_t)((long)min(TN, N - n0) * K * 2));
  // per-thread load slots (four 16-byte vectors of A and of B per K step)
  uint32_t oa[4], ob[4];
  int la[4], lb[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int v = tid + NT * u;
    const int r = v >> 3, c8 = (v & 7) * 8;          // [row][k]: 128 rows x 8 vectors
    oa[u] = (uint32_t)((r * K + c8) * 2);
    la[u] = r * PA + c8;
    if constexpr (NN) {                              // [k][n]: 64 rows x 16 vectors
      const int rk = v >> 4, cn = (v & 15) * 8;
      ob[u] = n0 + cn < N ? (uint32_t)((rk * N + cn) * 2) : kOob;
      lb[u] = rk * PB + cn;
    } else {
      ob[u] = (uint32_t)((r * K + c8) * 2);
      lb[u] = r * PA + c8;
    }
  }
  // K step s: A columns / NT rows' columns kk = 64 s + c8 (masked past K); NN rows kk = 64 s + rk
  auto gload = [&](u32x4v (&pa)[4], u32x4v (&pb)[4], int s) {
    const int kk = KS * s;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c8 = ((tid + NT * u) & 7) * 8;
      pa[u] = bld16(ra, kk + c8 < K ? oa[u] + (uint32_t)(kk * 2) : kOob);
      if constexpr (NN) pb[u] = bld16(rb, ob[u] == kOob ? kOob : ob[u] + (uint32_t)(kk * N * 2));
      else pb[u] = bld16(rb, kk + c8 < K ? ob[u] + (uint32_t)(kk * 2) : kOob);
    }
  };
  auto lstore = [&](const u32x4v (&pa)[4], const u32x4v (&pb)[4], int buf) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      *reinterpret_cast<u32x4v*>(&sm.a[buf][0][0] + la[u]) = pa[u];
      *reinterpret_cast<u32x4v*>(&sm.b[buf][0][0] + lb[u]) = pb[u];
    }
  };
  f32x4 acc[4][4];   // [n tile][m tile]: C^T
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[ct][mt] = zero4();

  const int nk = (K + KS - 1) / KS;
  u32x4v pa[4], pb[4];
  gload(pa, pb, 0);
  lstore(pa, pb, 0);
  if (nk > 1) gload(pa, pb, 1);
  __syncthreads();
  for (int s = 0; s < nk; ++s) {
    const int buf = s & 1;
#pragma unroll
    for (int ks = 0; ks < KS / 32; ++ks) {
      bf16x8 fb[4], fa[4];
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        if constexpr (NN) fb[ct] = frag_tr_l(&sm.b[buf][0][0], PB, 64 * wn + 16 * ct, 32 * ks, lane);
        else fb[ct] = frag_row(&sm.b[buf][0][0], PA, 64 * wn + 16 * ct, 32 * ks);
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) fa[mt] = frag_row(&sm.a[buf][0][0], PA, 64 * wm + 16 * mt, 32 * ks);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) acc[ct][mt] = mma_bf16(fb[ct], fa[mt], acc[ct][mt]);
    }
    if (s + 1 < nk) {   // the other buffer's reads ended before the last barrier
      lstore(pa, pb, buf ^ 1);
      if (s + 2 < nk) gload(pa, pb, s + 2);
    }
    __syncthreads();
  }
  // one unconditional product per accumulator after the runtime loop (see the rule in mem_common.h)
  const bf16x8 zf = zero_frag();
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[ct][mt] = mma_bf16(zf, zf, acc[ct][mt]);

  // lane (g, i) of tile (ct, mt): C[m0 + 64 wm + 16 mt + i][n0 + 64 wn + 16 ct + 4 g + r], r < 4
  const int g = lane >> 4, i = lane & 15;
  const rsrc_t rc = make_rsrc(p.c[z] + m0 * N, (uint32_t)(mrows * N * 2));
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const int n = 64 * wn + 16 * ct + 4 * g;
    if (n0 + n >= N) continue;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int m = 64 * wm + 16 * mt + i;
      u32x2v o;
      o[0] = pack_bf16x2(acc[ct][mt][0], acc[ct][mt][1]);
      o[1] = pack_bf16x2(acc[ct][mt][2], acc[ct][mt][3]);
      bst8(rc, (uint32_t)((m * N + n0 + n) * 2), o);   // rows past M are dropped by the range check
    }
  }
}

}  // namespace atlas

extern "C" {

int atlas_linear_batch(int b_layout, int count, int64_t m, const int* n, const int* k, const void* const* a,
                       const void* const* b, void* const* c, void* stream) {
  using namespace atlas;
  if (b_layout != ATLAS_GEMM_NT && b_layout != ATLAS_GEMM_NN) return ATLAS_MEM_ERR_ARG;
  if (count < 1 || count > gm::MAXP) return ATLAS_MEM_ERR_SHAPE;
  if (!n || !k || !a || !b || !c) return ATLAS_MEM_ERR_NULL;
  if (m < 0 || m >= ((int64_t)1 << 31)) return ATLAS_MEM_ERR_SHAPE;
  gm::Batch p = {};
  int nmax = 0;
  for (int z = 0; z < count; ++z) {
    if (n[z] < 8 || k[z] < 8 || n[z] % 8 || k[z] % 8 || n[z] > 65536 || k[z] > 65536) return ATLAS_MEM_ERR_SHAPE;
    // one workgroup's rows of A and C, and all of B, within a buffer resource's 32-bit range
    if ((int64_t)gm::TM * (k[z] > n[z] ? k[z] : n[z]) * 2 >= ((int64_t)1 << 31) ||
        (int64_t)k[z] * n[z] * 2 >= ((int64_t)1 << 31))
      return ATLAS_MEM_ERR_SHAPE;
    if (m > 0 && (!a[z] || !b[z] || !c[z])) return ATLAS_MEM_ERR_NULL;
    for (const void* q : {a[z], b[z], (const void*)c[z]})
      if (reinterpret_cast<uintptr_t>(q) & 15) return ATLAS_MEM_ERR_ALIGN;
    p.a[z] = static_cast<const bf16*>(a[z]);
    p.b[z] = static_cast<const bf16*>(b[z]);
    p.c[z] = static_cast<bf16*>(c[z]);
    p.n[z] = n[z];
    p.k[z] = k[z];
    nmax = n[z] > nmax ? n[z] : nmax;
  }
  if (m == 0) return ATLAS_MEM_OK;
  const dim3 grid((unsigned)((m + gm::TM - 1) / gm::TM), (unsigned)((nmax + gm::TN - 1) / gm::TN), (unsigned)count);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (b_layout == ATLAS_GEMM_NN)
    hipLaunchKernelGGL(k_gemm<true>, grid, dim3(gm::NT), 0, s, (long)m, p);
  else
    hipLaunchKernelGGL(k_gemm<false>, grid, dim3(gm::NT), 0, s, (long)m, p);
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

}  // extern "C"
