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
constexpr int MAXP = 4;           // problems per launch (sharing the token count)
struct Batch {
  const bf16* dy[MAXP];
  const bf16* x[MAXP];
  float* part[MAXP];
  void* dw[MAXP];
  int O[MAXP], I[MAXP], kc[MAXP], ntile[MAXP], S[MAXP];
  int off[MAXP + 1];              // first workgroup (k_wgrad) of each problem
  int roff[MAXP + 1];             // first partial float4 of one split (k_wgrad_reduce) of each problem
  int count;
};
// the problem of flattened index v given the cumulative starts (workgroup-uniform in k_wgrad)
__device__ __forceinline__ int batch_problem(const int (&off)[MAXP + 1], int count, long v) {
  int z = 0;
  while (z + 1 < count && v >= off[z + 1]) ++z;
  return z;
}
}  // namespace wg

// One workgroup per (problem, split, tile), flattened: problem z owns workgroups off[z] ..
// off[z + 1] - 1, local index = s ntile + tile with tile = to + nto ti; split s covers tokens
// [s kc, min(n, (s + 1) kc)).
__global__ __launch_bounds__(wg::NT) void k_wgrad(long n, wg::Batch bt) {
  using namespace wg;
  __shared__ Smem sm;
  const int tid = threadIdx.x, lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int z = batch_problem(bt.off, bt.count, blockIdx.x);
  const int O = bt.O[z], I = bt.I[z], kc = bt.kc[z], ntile = bt.ntile[z];
  const bf16* __restrict__ dy = bt.dy[z];
  const bf16* __restrict__ x = bt.x[z];
  const int local = blockIdx.x - bt.off[z];
  const int nto = (O + TILE - 1) / TILE;
  const int tile = local % ntile, s = local / ntile;
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
  const bf16x8 zf = zero_frag();
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = mma_bf16(zf, zf, acc[a][b]);

  // partial [s][tile][wave][a][b][lane] as float4: lane l of tile (a, b) holds
  // dW[o0 + 64 wo + 16 a + 4 (l >> 4) + r][i0 + 64 wi + 16 b + (l & 15)], r < 4
  float4* dst = reinterpret_cast<float4*>(bt.part[z]) + (((size_t)s * ntile + tile) * 4 + w) * 16 * FRAG4;
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
      dst[(a * 4 + b) * FRAG4 + lane] = make_float4(acc[a][b][0], acc[a][b][1], acc[a][b][2], acc[a][b][3]);
}

// dW from the S partials of k_wgrad, summed in split order; one thread per partial float4 of one
// split, flattened over the problems (problem z owns roff[z] .. roff[z + 1] - 1).
template <typename T>
__global__ __launch_bounds__(256) void k_wgrad_reduce(wg::Batch bt) {
  using namespace wg;
  const long v = (long)blockIdx.x * 256 + threadIdx.x;
  if (v >= bt.roff[bt.count]) return;
  const int z = batch_problem(bt.roff, bt.count, v);
  const long idx = v - bt.roff[z];
  const int O = bt.O[z], I = bt.I[z], S = bt.S[z];
  const long per = (long)bt.ntile[z] * (WG_FLOATS / 4);   // float4 per split
  const float4* p = reinterpret_cast<const float4*>(bt.part[z]) + idx;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);   // S = 0 (no tokens): dW = 0
#pragma unroll 8
  for (int s = 0; s < S; ++s) {   // unrolled so that the loads are in flight together; summed in order
    const float4 q = p[(size_t)s * per];
    acc.x += q.x; acc.y += q.y; acc.z += q.z; acc.w += q.w;
  }
  const int lane = (int)(idx & 63), ab = (int)((idx >> 6) & 15), w = (int)((idx >> 10) & 3);
  const int tile = (int)(idx >> 12);
  const int nto = (O + TILE - 1) / TILE;
  const int o = TILE * (tile % nto) + 64 * (w & 1) + 16 * (ab >> 2) + 4 * (lane >> 4);
  const int i = TILE * (tile / nto) + 64 * (w >> 1) + 16 * (ab & 3) + (lane & 15);
  if (i >= I) return;
  T* dw = static_cast<T*>(bt.dw[z]);
  const float val[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
  for (int r = 0; r < 4; ++r)
    if (o + r < O) dw[(size_t)(o + r) * I + i] = from_f32<T>(val[r]);
}

namespace {
bool wgrad_dims_ok(int64_t n, int o, int i) {
  return n >= 0 && n < ((int64_t)1 << 31) && o >= 8 && i >= 8 && o % 8 == 0 && i % 8 == 0 && o <= 65536 &&
         i <= 65536;
}
// Token chunk per split, common to the batch: about 256 workgroups for one problem (one per CU),
// 512 for a batch, at least 256 tokens (8 K steps) per workgroup. Returns false past the limits.
bool wgrad_plan(int count, int64_t n, const int* o, const int* i, wg::Batch& bt, int64_t& ws_bytes) {
  if (count < 1 || count > wg::MAXP) return false;
  int64_t tiles = 0;
  for (int z = 0; z < count; ++z) {
    if (!wgrad_dims_ok(n, o[z], i[z])) return false;
    bt.ntile[z] = ((o[z] + wg::TILE - 1) / wg::TILE) * ((i[z] + wg::TILE - 1) / wg::TILE);
    tiles += bt.ntile[z];
  }
  const int64_t target = count > 1 ? 512 : 256;
  const int64_t s_target = tiles >= target ? 1 : target / tiles;
  int64_t kc = (n + s_target - 1) / s_target;
  kc = ((kc + wg::KS - 1) / wg::KS) * wg::KS;
  if (kc < 256) kc = 256;
  const int S = n == 0 ? 0 : (int)((n + kc - 1) / kc);
  bt.count = count;
  ws_bytes = 0;
  int64_t wgs = 0, r4 = 0;
  for (int z = 0; z < count; ++z) {
    if (kc * (o[z] > i[z] ? o[z] : i[z]) * 2 >= ((int64_t)1 << 30)) return false;
    bt.O[z] = o[z];
    bt.I[z] = i[z];
    bt.kc[z] = (int)kc;
    bt.S[z] = S;
    bt.off[z] = (int)wgs;
    bt.roff[z] = (int)r4;
    wgs += (int64_t)S * bt.ntile[z];
    r4 += (int64_t)bt.ntile[z] * (wg::WG_FLOATS / 4);
    ws_bytes += (int64_t)S * bt.ntile[z] * wg::WG_FLOATS * (int64_t)sizeof(float);
    if (wgs >= ((int64_t)1 << 30) || r4 >= ((int64_t)1 << 30)) return false;
  }
  bt.off[count] = (int)wgs;
  bt.roff[count] = (int)r4;
  return true;
}
}  // namespace

}  // namespace atlas

extern "C" {

int64_t atlas_linear_wgrad_batch_workspace_bytes(int count, int64_t n, const int* out_features,
                                                 const int* in_features) {
  if (!out_features || !in_features) return -1;
  atlas::wg::Batch bt = {};
  int64_t bytes = 0;
  return atlas::wgrad_plan(count, n, out_features, in_features, bt, bytes) ? bytes : -1;
}

int atlas_linear_wgrad_batch(int out_dtype, int count, int64_t n, const int* out_features, const int* in_features,
                             const void* const* dy, const void* const* x, void* const* dw, void* workspace,
                             int64_t workspace_bytes, void* stream) {
  using namespace atlas;
  if (out_dtype != ATLAS_DT_BF16 && out_dtype != ATLAS_DT_F32) return ATLAS_MEM_ERR_DTYPE;
  if (!out_features || !in_features || !dy || !x || !dw) return ATLAS_MEM_ERR_NULL;
  wg::Batch bt = {};
  int64_t need = 0;
  if (!wgrad_plan(count, n, out_features, in_features, bt, need)) return ATLAS_MEM_ERR_SHAPE;
  if (n > 0 && !workspace) return ATLAS_MEM_ERR_NULL;
  if (reinterpret_cast<uintptr_t>(workspace) & 15) return ATLAS_MEM_ERR_ALIGN;
  if (workspace_bytes < need) return ATLAS_MEM_ERR_WORKSPACE;
  float* part = static_cast<float*>(workspace);
  for (int z = 0; z < count; ++z) {
    if (!dw[z] || (n > 0 && (!dy[z] || !x[z]))) return ATLAS_MEM_ERR_NULL;   // n = 0 reads no operand
    if ((reinterpret_cast<uintptr_t>(dy[z]) & 15) || (reinterpret_cast<uintptr_t>(x[z]) & 15))
      return ATLAS_MEM_ERR_ALIGN;
    bt.dy[z] = static_cast<const bf16*>(dy[z]);
    bt.x[z] = static_cast<const bf16*>(x[z]);
    bt.dw[z] = dw[z];
    bt.part[z] = part;
    part += (size_t)bt.S[z] * bt.ntile[z] * wg::WG_FLOATS;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (bt.off[count] > 0) hipLaunchKernelGGL(k_wgrad, dim3(bt.off[count]), dim3(wg::NT), 0, s, (long)n, bt);
  const unsigned rgrid = (unsigned)((bt.roff[count] + 255) / 256);
  if (out_dtype == ATLAS_DT_F32) hipLaunchKernelGGL(k_wgrad_reduce<float>, dim3(rgrid), dim3(256), 0, s, bt);
  else hipLaunchKernelGGL(k_wgrad_reduce<bf16>, dim3(rgrid), dim3(256), 0, s, bt);
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

int64_t atlas_linear_wgrad_workspace_bytes(int64_t n, int out_features, int in_features) {
  return atlas_linear_wgrad_batch_workspace_bytes(1, n, &out_features, &in_features);
}

int atlas_linear_wgrad(int out_dtype, int64_t n, int out_features, int in_features, const void* dy, const void* x,
                       void* dw, void* workspace, int64_t workspace_bytes, void* stream) {
  return atlas_linear_wgrad_batch(out_dtype, 1, n, &out_features, &in_features, &dy, &x, &dw, workspace,
                                  workspace_bytes, stream);
}

}  // extern "C"
