// wgrad.hip - weight gradient of a bias-free linear layer over the tokens, dW = dy^T x, for bf16
// row-major activations: the backward of the cell's projections (LinearNoBias to_q / to_k / to_v /
// to_out, rnn_memory.py:486-489, and the gate heads' Linear(dim, heads), :503-520), whose weight
// gradients autograd forms from the same two tensors.
//
//   dy [N, O], x [N, I] (row-major, as the forward and the head-split adjoint leave them)
//   dW [O, I] = sum_n dy[n, :]^T x[n, :]                     (fp32 accumulate, bf16 or fp32 out)
//
// Neither operand is copied into a transposed layout: a K step stages 32 token rows of the
// workgroup's 128 dy columns and 128 x columns in LDS as stored, and both matrix-core operands are
// read transposed from there (ds_read_b64_tr_b16), so that v_mfma_f32_16x16x32_bf16 runs over the
// tokens. The output has few 128 x 128 tiles while K = N is long (16384 tokens at the cell's
// shapes), so the token axis is split S ways; each workgroup stores its fp32 tile in the
// accumulator's own fragment order (one 16-byte store per lane and 16 x 16 tile) and
// k_wgrad_reduce sums the S partials in a fixed order (deterministic) into dW.
#include "../../include/atlas_mem.h"
#include "mem_common.h"
#include "walk_common.h"

namespace atlas {

namespace wg {
constexpr int TILE = 128;        // output tile (o and i)
constexpr int KS = 32;           // tokens per K step
constexpr int P = TILE + 16;     // LDS pitch: the four rows of a transposing read hit distinct banks
constexpr int NT = 256;          // 4 waves, 2 x 2 over the tile, 64 x 64 (4 x 4 MFMA tiles) each
constexpr int FRAG4 = 64;        // float4 per 16 x 16 accumulator tile (one per lane)
constexpr int WG_FLOATS = TILE * TILE;
struct Smem {
  alignas(16) bf16 a[2][KS][P];   // dy rows of the K step (columns o0 ..), by step parity
  alignas(16) bf16 b[2][KS][P];   // x rows (columns i0 ..)
};
}  // namespace wg

// grid (tiles, S): tile = to + nto * ti; split s covers tokens [s kc, min(n, (s + 1) kc))
__global__ __launch_bounds__(wg::NT) void k_wgrad(long n, int O, int I, int kc, const bf16* __restrict__ dy,
                                                  const bf16* __restrict__ x, float* __restrict__ part) {
  using namespace wg;
  __shared__ Smem sm;
  const int tid = threadIdx.x, lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nto = (O + TILE - 1) / TILE;
  const int tile = blockIdx.x, s = blockIdx.y;
  const int o0 = TILE * (tile % nto), i0 = TILE * (tile / nto);
  const long t0 = (long)s * kc;
  const long nrows = min((long)kc, n - t0);
  // rows past the split's end read zeros (buffer range); columns past O / I read zeros (kOob)
  const rsrc_t ra = make_rsrc(dy + t0 * O, (uint32_t)(nrows * O * 2));
  const rsrc_t rb = make_rsrc(x + t0 * I, (uint32_t)(nrows * I * 2));
  const int lr = tid >> 4, lc = tid & 15;   // rows lr, lr + 16 of the step; columns 8 lc .. 8 lc + 7
  const uint32_t oa = o0 + 8 * lc < O ? (uint32_t)((lr * O + o0 + 8 * lc) * 2) : kOob;
  const uint32_t ob = i0 + 8 * lc < I ? (uint32_t)((lr * I + i0 + 8 * lc) * 2) : kOob;
  const uint32_t sa = (uint32_t)(KS * O * 2), sb = (uint32_t)(KS * I * 2);
  // register stages of the K steps ahead (three, so that two steps' loads are in flight while the
  // third is stored to LDS); steps past the split's end read zeros and add nothing
  struct Stage {
    u32x4v a0, a1, b0, b1;
  };
  auto gload = [&](Stage& st, int k) {
    st.a0 = bld16(ra, oa + (uint32_t)k * sa);
    st.a1 = bld16(ra, oa + (uint32_t)k * sa + (uint32_t)(16 * O * 2));
    st.b0 = bld16(rb, ob + (uint32_t)k * sb);
    st.b1 = bld16(rb, ob + (uint32_t)k * sb + (uint32_t)(16 * I * 2));
  };
  auto lstore = [&](const Stage& st, int buf) {
    *reinterpret_cast<u32x4v*>(&sm.a[buf][lr][8 * lc]) = st.a0;
    *reinterpret_cast<u32x4v*>(&sm.a[buf][lr + 16][8 * lc]) = st.a1;
    *reinterpret_cast<u32x4v*>(&sm.b[buf][lr][8 * lc]) = st.b0;
    *reinterpret_cast<u32x4v*>(&sm.b[buf][lr + 16][8 * lc]) = st.b1;
  };
  const int wo = w & 1, wi = w >> 1;
  f32x4 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = zero4();

  // step k: products of LDS buffer k & 1; then the stage holding step k + 1 goes to the other
  // buffer (whose reads ended before the last barrier) and is refilled with step k + 4
  auto step = [&](int k, Stage& st) {
    const int buf = k & 1;
    bf16x8 fa[4], fb[4];
#pragma unroll
    for (int a = 0; a < 4; ++a) fa[a] = frag_tr_l(&sm.a[buf][0][0], P, 64 * wo + 16 * a, 0, lane);
#pragma unroll
    for (int b = 0; b < 4; ++b) fb[b] = frag_tr_l(&sm.b[buf][0][0], P, 64 * wi + 16 * b, 0, lane);
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) acc[a][b] = mma_bf16(fa[a], fb[b], acc[a][b]);
    lstore(st, buf ^ 1);
    gload(st, k + 4);
    __syncthreads();
  };
  const int nk = (int)((nrows + KS - 1) / KS);
  Stage s0, s1, s2;
  gload(s0, 0);
  lstore(s0, 0);
  gload(s0, 1);
  gload(s1, 2);
  gload(s2, 3);
  __syncthreads();
  for (int k = 0; k < nk; k += 3) {   // up to two trailing steps of zeros
    step(k, s0);
    step(k + 1, s1);
    step(k + 2, s2);
  }
  // one unconditional product per accumulator after the runtime loop (see the rule in mem_common.h)
  const bf16x8 z = zero_frag();
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = mma_bf16(z, z, acc[a][b]);

  // partial [s][tile][wave][a][b][lane] as float4: lane l of tile (a, b) holds
  // dW[o0 + 64 wo + 16 a + 4 (l >> 4) + r][i0 + 64 wi + 16 b + (l & 15)], r < 4
  const int ntile = gridDim.x;
  float4* dst = reinterpret_cast<float4*>(part) + (((size_t)s * ntile + tile) * 4 + w) * 16 * FRAG4;
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
      dst[(a * 4 + b) * FRAG4 + lane] = make_float4(acc[a][b][0], acc[a][b][1], acc[a][b][2], acc[a][b][3]);
}

// dW from the S partials of k_wgrad, summed in split order; one thread per partial float4.
template <typename T>
__global__ __launch_bounds__(256) void k_wgrad_reduce(int O, int I, int S, int ntile, const float* __restrict__ part,
                                                      T* __restrict__ dw) {
  using namespace wg;
  const long per = (long)ntile * (WG_FLOATS / 4);   // float4 per split
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= per) return;
  const float4* p = reinterpret_cast<const float4*>(part) + idx;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);   // S = 0 (no tokens): dW = 0
#pragma unroll 8
  for (int s = 0; s < S; ++s) {   // unrolled so that the loads are in flight together; summed in order
    const float4 v = p[(size_t)s * per];
    acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
  }
  const int lane = (int)(idx & 63), ab = (int)((idx >> 6) & 15), w = (int)((idx >> 10) & 3);
  const int tile = (int)(idx >> 12);
  const int nto = (O + TILE - 1) / TILE;
  const int o = TILE * (tile % nto) + 64 * (w & 1) + 16 * (ab >> 2) + 4 * (lane >> 4);
  const int i = TILE * (tile / nto) + 64 * (w >> 1) + 16 * (ab & 3) + (lane & 15);
  if (i >= I) return;
  const float v[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
  for (int r = 0; r < 4; ++r)
    if (o + r < O) dw[(size_t)(o + r) * I + i] = from_f32<T>(v[r]);
}

namespace {
struct WgradPlan {
  int ntile, S, kc;
};
// Token chunk per split: about 256 workgroups over the output tiles (one per CU), at least 256
// tokens (8 K steps) per workgroup.
WgradPlan wgrad_plan(int64_t n, int o, int i) {
  WgradPlan p;
  p.ntile = ((o + wg::TILE - 1) / wg::TILE) * ((i + wg::TILE - 1) / wg::TILE);
  const int64_t s_target = p.ntile >= 256 ? 1 : 256 / p.ntile;
  int64_t kc = (n + s_target - 1) / s_target;
  kc = ((kc + wg::KS - 1) / wg::KS) * wg::KS;
  if (kc < 256) kc = 256;
  p.kc = (int)kc;
  p.S = (int)((n + kc - 1) / kc);
  return p;
}
bool wgrad_dims_ok(int64_t n, int o, int i) {
  return n >= 0 && n < ((int64_t)1 << 31) && o >= 8 && i >= 8 && o % 8 == 0 && i % 8 == 0 && o <= 65536 &&
         i <= 65536;
}
}  // namespace

}  // namespace atlas

extern "C" {

int64_t atlas_linear_wgrad_workspace_bytes(int64_t n, int out_features, int in_features) {
  if (!atlas::wgrad_dims_ok(n, out_features, in_features)) return -1;
  if (n == 0) return 0;
  const atlas::WgradPlan p = atlas::wgrad_plan(n, out_features, in_features);
  return (int64_t)p.S * p.ntile * atlas::wg::WG_FLOATS * (int64_t)sizeof(float);
}

int atlas_linear_wgrad(int out_dtype, int64_t n, int out_features, int in_features, const void* dy, const void* x,
                       void* dw, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace atlas;
  if (out_dtype != ATLAS_DT_BF16 && out_dtype != ATLAS_DT_F32) return ATLAS_MEM_ERR_DTYPE;
  if (!wgrad_dims_ok(n, out_features, in_features)) return ATLAS_MEM_ERR_SHAPE;
  if (!dw || (n > 0 && (!dy || !x || !workspace))) return ATLAS_MEM_ERR_NULL;   // n = 0 reads no operand
  if ((reinterpret_cast<uintptr_t>(dy) & 15) || (reinterpret_cast<uintptr_t>(x) & 15) ||
      (reinterpret_cast<uintptr_t>(workspace) & 15))
    return ATLAS_MEM_ERR_ALIGN;
  const int O = out_features, I = in_features;
  hipStream_t s = static_cast<hipStream_t>(stream);
  WgradPlan p = wgrad_plan(n, O, I);
  if (n == 0) p.S = 0;   // an empty sum: the reduce writes zeros and reads no partial
  if (workspace_bytes < (int64_t)p.S * p.ntile * wg::WG_FLOATS * (int64_t)sizeof(float)) return ATLAS_MEM_ERR_WORKSPACE;
  if ((int64_t)p.kc * (O > I ? O : I) * 2 >= ((int64_t)1 << 30)) return ATLAS_MEM_ERR_SHAPE;
  float* part = static_cast<float*>(workspace);
  if (p.S > 0)
    hipLaunchKernelGGL(k_wgrad, dim3(p.ntile, p.S), dim3(wg::NT), 0, s, (long)n, O, I, p.kc,
                       static_cast<const bf16*>(dy), static_cast<const bf16*>(x), part);
  const long per4 = (long)p.ntile * (wg::WG_FLOATS / 4);
  const unsigned rgrid = (unsigned)((per4 + 255) / 256);
  if (out_dtype == ATLAS_DT_F32)
    hipLaunchKernelGGL(k_wgrad_reduce<float>, dim3(rgrid), dim3(256), 0, s, O, I, p.S, p.ntile, part,
                       static_cast<float*>(dw));
  else
    hipLaunchKernelGGL(k_wgrad_reduce<bf16>, dim3(rgrid), dim3(256), 0, s, O, I, p.S, p.ntile, part,
                       static_cast<bf16*>(dw));
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

}  // extern "C"
