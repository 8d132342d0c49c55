// blocks.hip - the state-block decomposition of the recurrence for head sizes above the kernels'
// 64 (BASELINE C4: d_k = 128 after the tensor feature map, d_v = 64), fused.
//
// With S split into 64 x 64 blocks S[i, j] (rows 64 i of d_v, columns 64 j of d_k), the column blocks
// couple only through delta = S_ref phi - v; every block then runs the 64-wide recurrence with
// S_ref = 0 and v = -delta[rows of block i]. The blocks are stacked along the row axis as
// r = (i * nbk + j) * BH + bh (the host's order).
//   k_block_split : one pass over phi, psi, v: phi_b[r] = phi[:, 64 j ..], psi_b[r] = psi[:, 64 j ..],
//                   nv_b[r] = (v - S_ref phi)[:, 64 i ..], the product on the fp32 matrix cores
//   k_block_merge : its adjoint per token: dphi = sum_i dphi_b[(i, j)] | ... - S_ref^T dnv, dpsi likewise,
//                   dv = dnv = sum_j dnv_b[(i, j)]
//   k_block_dsref : per-256-token partials of dS_ref = -sum_t dnv_t phi_t^T, one workgroup per 64 x 64 block
// One workgroup (256 threads) per 64 tokens of one row (dS_ref: per 256 tokens and block); rows move in
// 16-byte vectors; LDS is sized by the blocks present (the merge's S_ref^T dnv reuses the S_ref tile).
#include <hip/hip_runtime.h>

#include "../../include/atlas_mem.h"
#include "mem_common.h"

namespace atlas {

namespace blk {
constexpr int kThreads = 256;
constexpr int TT = 64;            // tokens per tile
constexpr int B = 64;             // block width
constexpr int kPartTiles = 4;     // tiles per dS_ref partial (256 tokens)
constexpr int MaxD = 256;         // d_k, d_v <= 256
constexpr int P = B + 4;          // LDS pitch (fp32), 16-byte aligned rows
typedef MM<float> M;
}

__device__ __forceinline__ void lds8(float* s, const float* v) {
  reinterpret_cast<float4*>(s)[0] = make_float4(v[0], v[1], v[2], v[3]);
  reinterpret_cast<float4*>(s)[1] = make_float4(v[4], v[5], v[6], v[7]);
}

// rows x 64 values from a row-major [., ld] source into LDS s[rows][P] as fp32 (rows >= rows_real: zero).
template <typename T>
__device__ __forceinline__ void tile_in(float (*s)[blk::P], const T* src, int ld, int rows, int rows_real) {
  for (int u = threadIdx.x; u < rows * (blk::B / 8); u += blk::kThreads) {
    const int r = u / (blk::B / 8), c = (u % (blk::B / 8)) * 8;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (r < rows_real) ld8(src + (size_t)r * ld + c, v);
    lds8(&s[r][c], v);
  }
}

// phi, psi [BH, T, dk]; v [BH, T, dv]; S_ref [BH, dv, dk] fp32 -> phi_b, psi_b, nv_b [NB BH, T, 64].
template <typename T>
__global__ __launch_bounds__(blk::kThreads) void k_block_split(int BH, int Tn, int dk, int dv, const T* __restrict__ phi,
                                                               const T* __restrict__ psi, const T* __restrict__ v,
                                                               const float* __restrict__ S_ref, T* __restrict__ phi_b,
                                                               T* __restrict__ psi_b, T* __restrict__ nv_b) {
  using namespace blk;
  __shared__ __align__(16) float sx[TT][P];   // phi columns 64 kb .. of the tile; then S_ref phi of block i
  __shared__ __align__(16) float sr[B][P];    // S_ref rows 64 i .., columns 64 kb ..
  float (*sy)[P] = sx;
  const int t0 = blockIdx.x * TT, bh = blockIdx.y, tid = threadIdx.x, l = lane_id(), w = wave_id();
  const int nt = min(TT, Tn - t0);
  const int nbk = dk / B, nbv = dv / B;
  // the column blocks of phi and psi, copied once per (i, j) in 16-byte vectors
  for (int j = 0; j < nbk; ++j)
    for (int u = tid; u < nt * (B / 8); u += blk::kThreads) {
      const int t = u / (B / 8), c8 = (u % (B / 8)) * 8;
      const size_t src = ((size_t)bh * Tn + t0 + t) * dk + j * B + c8;
      float a[8], b[8];
      ld8(phi + src, a);
      ld8(psi + src, b);
      for (int i = 0; i < nbv; ++i) {
        const size_t dst = (((size_t)(i * nbk + j) * BH + bh) * Tn + t0 + t) * B + c8;
        st8(phi_b + dst, a);
        st8(psi_b + dst, b);
      }
    }
  // nv = v - S_ref phi, one 64-row block i at a time: C[t][a] over k in 64-wide column blocks
  for (int i = 0; i < nbv; ++i) {
    f32x4 acc[4];   // wave w: tokens 16 w .. x value tiles n
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[n] = zero4();
    for (int kb = 0; kb < nbk; ++kb) {
      __syncthreads();
      tile_in(sx, phi + ((size_t)bh * Tn + t0) * dk + kb * B, dk, TT, nt);
      tile_in(sr, S_ref + ((size_t)bh * dv + i * B) * dk + kb * B, dk, B, B);
      __syncthreads();
#pragma unroll
      for (int n = 0; n < 4; ++n)
        for (int k0 = 0; k0 < B; k0 += 4)
          acc[n] = M::mma(sx[16 * w + (l & 15)][k0 + (l >> 4)], sr[16 * n + (l & 15)][k0 + (l >> 4)], acc[n]);
    }
    __syncthreads();   // sy aliases sx
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int q = 0; q < 4; ++q) sy[16 * w + 4 * (l >> 4) + q][16 * n + (l & 15)] = acc[n][q];
    __syncthreads();
    for (int u = tid; u < nt * (B / 8); u += blk::kThreads) {
      const int t = u / (B / 8), c8 = (u % (B / 8)) * 8;
      float x[8];
      ld8(v + ((size_t)bh * Tn + t0 + t) * dv + i * B + c8, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] -= sy[t][c8 + e];
      for (int j = 0; j < nbk; ++j) st8(nv_b + (((size_t)(i * nbk + j) * BH + bh) * Tn + t0 + t) * B + c8, x);
    }
  }
}

// Adjoint of k_block_split per 64-token tile: dv = dnv = sum_j dnv_b[(i, j)], dpsi = sum_i dpsi_b[(i, j)],
// dphi = sum_i dphi_b[(i, j)] - S_ref^T dnv.
template <typename T>
__global__ __launch_bounds__(blk::kThreads) void k_block_merge(int BH, int Tn, int dk, int dv,
                                                               const float* __restrict__ S_ref,
                                                               const T* __restrict__ dphi_b, const T* __restrict__ dpsi_b,
                                                               const T* __restrict__ dnv_b, T* __restrict__ dphi,
                                                               T* __restrict__ dpsi, T* __restrict__ dv_out) {
  using namespace blk;
  // dynamic LDS: sd[nbv][TT][P] (dnv of the tile, every value block i), then sr[B][P] (S_ref block
  // (i, kb)), which sk[TT][P] ((S_ref^T dnv)[t][kb block]) reuses once the block's products are done
  extern __shared__ __align__(16) float blk_smem[];
  const int t0 = blockIdx.x * TT, bh = blockIdx.y, tid = threadIdx.x, l = lane_id(), w = wave_id();
  const int nt = min(TT, Tn - t0);
  const int nbk = dk / B, nbv = dv / B;
  float (*sd)[TT][P] = reinterpret_cast<float (*)[TT][P]>(blk_smem);
  float (*sr)[P] = reinterpret_cast<float (*)[P]>(blk_smem + (size_t)nbv * TT * P);
  float (*sk)[P] = sr;
  auto row = [&](int i, int j, int t) { return (((size_t)(i * nbk + j) * BH + bh) * Tn + t0 + t) * B; };
  for (int i = 0; i < nbv; ++i)
    for (int u = tid; u < TT * (B / 8); u += blk::kThreads) {
      const int t = u / (B / 8), c8 = (u % (B / 8)) * 8;
      float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (t < nt) {
        for (int j = 0; j < nbk; ++j) {
          float x[8];
          ld8(dnv_b + row(i, j, t) + c8, x);
#pragma unroll
          for (int e = 0; e < 8; ++e) s[e] += x[e];
        }
        st8(dv_out + ((size_t)bh * Tn + t0 + t) * dv + i * B + c8, s);
      }
      lds8(&sd[i][t][c8], s);
    }
  for (int j = 0; j < nbk; ++j)
    for (int u = tid; u < nt * (B / 8); u += blk::kThreads) {
      const int t = u / (B / 8), c8 = (u % (B / 8)) * 8;
      float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int i = 0; i < nbv; ++i) {
        float x[8];
        ld8(dpsi_b + row(i, j, t) + c8, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) s[e] += x[e];
      }
      st8(dpsi + ((size_t)bh * Tn + t0 + t) * dk + j * B + c8, s);
    }
  for (int kb = 0; kb < nbk; ++kb) {
    f32x4 acc[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[n] = zero4();
    for (int i = 0; i < nbv; ++i) {
      __syncthreads();
      tile_in(sr, S_ref + ((size_t)bh * dv + i * B) * dk + kb * B, dk, B, B);
      __syncthreads();
      // (S_ref^T dnv)[t][c] = sum_a dnv[t][a] S_ref[a][c]
#pragma unroll
      for (int n = 0; n < 4; ++n)
        for (int k0 = 0; k0 < B; k0 += 4)
          acc[n] = M::mma(sd[i][16 * w + (l & 15)][k0 + (l >> 4)], sr[k0 + (l >> 4)][16 * n + (l & 15)], acc[n]);
    }
    __syncthreads();   // sk aliases sr
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int q = 0; q < 4; ++q) sk[16 * w + 4 * (l >> 4) + q][16 * n + (l & 15)] = acc[n][q];
    __syncthreads();
    for (int u = tid; u < nt * (B / 8); u += blk::kThreads) {
      const int t = u / (B / 8), c8 = (u % (B / 8)) * 8;
      float s[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) s[e] = -sk[t][c8 + e];
      for (int i = 0; i < nbv; ++i) {
        float x[8];
        ld8(dphi_b + row(i, kb, t) + c8, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) s[e] += x[e];
      }
      st8(dphi + ((size_t)bh * Tn + t0 + t) * dk + kb * B + c8, s);
    }
  }
}

// dS_ref partials: part p of row bh covers tokens [256 p, 256 p + 256): out[a][c] = -sum_t dv[t][a] phi[t][c]
// (dv: the merged dnv) for the 64 x 64 block (i, kb) = blockIdx.z; wave w owns value rows 16 w ..
template <typename T>
__global__ __launch_bounds__(blk::kThreads) void k_block_dsref(int BH, int Tn, int dk, int dv, const T* __restrict__ phi,
                                                               const T* __restrict__ dvv, float* __restrict__ part) {
  using namespace blk;
  __shared__ __align__(16) float sd[TT][P];
  __shared__ __align__(16) float sx[TT][P];
  const int p = blockIdx.x, bh = blockIdx.y, l = lane_id(), w = wave_id();
  const int nbk = dk / B, n_parts = gridDim.x;
  const int i = blockIdx.z / nbk, kb = blockIdx.z % nbk;
  f32x4 acc[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) acc[n] = zero4();
  for (int tile = 0; tile < kPartTiles; ++tile) {
    const int t0 = (p * kPartTiles + tile) * TT;
    if (t0 >= Tn) break;   // workgroup-uniform
    const int nt = min(TT, Tn - t0);
    __syncthreads();
    tile_in(sd, dvv + ((size_t)bh * Tn + t0) * dv + i * B, dv, TT, nt);
    tile_in(sx, phi + ((size_t)bh * Tn + t0) * dk + kb * B, dk, TT, nt);
    __syncthreads();
#pragma unroll
    for (int n = 0; n < 4; ++n)
      for (int k0 = 0; k0 < TT; k0 += 4)
        acc[n] = M::mma(sd[k0 + (l >> 4)][16 * w + (l & 15)], sx[k0 + (l >> 4)][16 * n + (l & 15)], acc[n]);
  }
  float* dst = part + ((size_t)bh * n_parts + p) * dv * dk;
#pragma unroll
  for (int n = 0; n < 4; ++n)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      dst[(size_t)(i * B + 16 * w + 4 * (l >> 4) + q) * dk + kb * B + 16 * n + (l & 15)] = -acc[n][q];
}

// The per-token scalars shared by every block, replicated along the stacked row axis, and the
// adjoint: the sum over the replicas. Up to four arrays per launch, 8 elements per thread (16-byte
// accesses when the array allows them), fp32 sums in replica order 0, 1, ... (deterministic).
namespace rep {
constexpr int kMax = 4, kThreads = 256, kVec = 8;
struct List {
  const void* src[kMax];
  void* dst[kMax];
  long n[kMax];
  long off[kMax + 1];   // first thread of each array (n / 8 rounded up)
  int vec[kMax];        // both arrays 16-byte aligned, n % 8 == 0: vector accesses
  int count, nrep;
};
}  // namespace rep

template <typename T, bool SUM>
__global__ __launch_bounds__(rep::kThreads) void k_replicas(rep::List L) {
  const long v = (long)blockIdx.x * rep::kThreads + threadIdx.x;
  if (v >= L.off[L.count]) return;
  int z = 0;
  while (z + 1 < L.count && v >= L.off[z + 1]) ++z;
  const long i0 = (v - L.off[z]) * rep::kVec, n = L.n[z];
  const T* src = static_cast<const T*>(L.src[z]);
  T* dst = static_cast<T*>(L.dst[z]);
  constexpr int PER16 = 16 / sizeof(T);   // elements per 16-byte access
  struct alignas(16) V { T e[PER16]; };   // one 16-byte access, moved as a whole vector
  if (L.vec[z]) {
    typedef float f32x4v __attribute__((ext_vector_type(4)));
    if constexpr (SUM) {
      float acc[rep::kVec] = {};
      for (int r = 0; r < L.nrep; ++r) {
#pragma unroll
        for (int h = 0; h < rep::kVec / PER16; ++h) {
          const V x = __builtin_bit_cast(V, *reinterpret_cast<const f32x4v*>(src + (size_t)r * n + i0 + h * PER16));
#pragma unroll
          for (int u = 0; u < PER16; ++u) acc[h * PER16 + u] += to_f32(x.e[u]);
        }
      }
#pragma unroll
      for (int h = 0; h < rep::kVec / PER16; ++h) {
        V o;
#pragma unroll
        for (int u = 0; u < PER16; ++u) o.e[u] = from_f32<T>(acc[h * PER16 + u]);
        *reinterpret_cast<f32x4v*>(dst + i0 + h * PER16) = __builtin_bit_cast(f32x4v, o);
      }
    } else {
      f32x4v x[rep::kVec / PER16];
#pragma unroll
      for (int h = 0; h < rep::kVec / PER16; ++h) x[h] = *reinterpret_cast<const f32x4v*>(src + i0 + h * PER16);
      for (int r = 0; r < L.nrep; ++r)
#pragma unroll
        for (int h = 0; h < rep::kVec / PER16; ++h)
          *reinterpret_cast<f32x4v*>(dst + (size_t)r * n + i0 + h * PER16) = x[h];
    }
    return;
  }
  const long i1 = n < i0 + rep::kVec ? n : i0 + rep::kVec;
  for (long i = i0; i < i1; ++i) {
    if constexpr (SUM) {
      float acc = 0.f;
      for (int r = 0; r < L.nrep; ++r) acc += to_f32(src[(size_t)r * n + i]);
      dst[i] = from_f32<T>(acc);
    } else {
      const T x = src[i];
      for (int r = 0; r < L.nrep; ++r) dst[(size_t)r * n + i] = x;
    }
  }
}

}  // namespace atlas

using namespace atlas;

namespace {
bool blk_dims_ok(int BH, int Tn, int dk, int dv) {
  return BH >= 1 && BH <= 65535 && Tn >= 1 && dk >= blk::B && dv >= blk::B && dk % blk::B == 0 && dv % blk::B == 0 &&
         dk <= blk::MaxD && dv <= blk::MaxD;
}
bool blk_misaligned(const void* p) { return p && (reinterpret_cast<uintptr_t>(p) & 15) != 0; }
}  // namespace

extern "C" {

int atlas_block_parts(int seq_len) {
  return seq_len < 1 ? 0 : (seq_len + blk::TT * blk::kPartTiles - 1) / (blk::TT * blk::kPartTiles);
}

int atlas_block_split(int dtype, int bh, int seq_len, int d_k, int d_v, const void* phi, const void* psi, const void* v,
                      const float* S_ref, void* phi_b, void* psi_b, void* nv_b, void* stream) {
  if (dtype != ATLAS_DT_F32 && dtype != ATLAS_DT_BF16) return ATLAS_MEM_ERR_DTYPE;
  if (!blk_dims_ok(bh, seq_len, d_k, d_v)) return ATLAS_MEM_ERR_SHAPE;
  if (!phi || !psi || !v || !S_ref || !phi_b || !psi_b || !nv_b) return ATLAS_MEM_ERR_NULL;
  for (const void* p : {phi, psi, v, (const void*)S_ref, (const void*)phi_b, (const void*)psi_b, (const void*)nv_b})
    if (blk_misaligned(p)) return ATLAS_MEM_ERR_ALIGN;
  const dim3 grid((seq_len + blk::TT - 1) / blk::TT, bh);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == ATLAS_DT_BF16)
    hipLaunchKernelGGL(k_block_split<bf16>, grid, dim3(blk::kThreads), 0, s, bh, seq_len, d_k, d_v, (const bf16*)phi,
                       (const bf16*)psi, (const bf16*)v, S_ref, (bf16*)phi_b, (bf16*)psi_b, (bf16*)nv_b);
  else
    hipLaunchKernelGGL(k_block_split<float>, grid, dim3(blk::kThreads), 0, s, bh, seq_len, d_k, d_v, (const float*)phi,
                       (const float*)psi, (const float*)v, S_ref, (float*)phi_b, (float*)psi_b, (float*)nv_b);
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

int atlas_block_merge(int dtype, int bh, int seq_len, int d_k, int d_v, const void* phi, const float* S_ref,
                      const void* dphi_b, const void* dpsi_b, const void* dnv_b, void* dphi, void* dpsi, void* dv,
                      float* dsref_part, void* stream) {
  if (dtype != ATLAS_DT_F32 && dtype != ATLAS_DT_BF16) return ATLAS_MEM_ERR_DTYPE;
  if (!blk_dims_ok(bh, seq_len, d_k, d_v)) return ATLAS_MEM_ERR_SHAPE;
  if (!phi || !S_ref || !dphi_b || !dpsi_b || !dnv_b || !dphi || !dpsi || !dv || !dsref_part) return ATLAS_MEM_ERR_NULL;
  for (const void* p : {phi, (const void*)S_ref, dphi_b, dpsi_b, dnv_b, (const void*)dphi, (const void*)dpsi,
                        (const void*)dv, (const void*)dsref_part})
    if (blk_misaligned(p)) return ATLAS_MEM_ERR_ALIGN;
  const dim3 grid((seq_len + blk::TT - 1) / blk::TT, bh), pgrid(atlas_block_parts(seq_len), bh, (d_v / blk::B) * (d_k / blk::B));
  const size_t smem = ((size_t)(d_v / blk::B) * blk::TT + blk::B) * blk::P * sizeof(float);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const void* mk = dtype == ATLAS_DT_BF16 ? reinterpret_cast<const void*>(&k_block_merge<bf16>)
                                          : reinterpret_cast<const void*>(&k_block_merge<float>);
  if (set_dyn_smem(mk, smem) != hipSuccess)
    return ATLAS_MEM_ERR_LAUNCH;
  if (dtype == ATLAS_DT_BF16) {
    hipLaunchKernelGGL(k_block_merge<bf16>, grid, dim3(blk::kThreads), smem, s, bh, seq_len, d_k, d_v, S_ref,
                       (const bf16*)dphi_b, (const bf16*)dpsi_b, (const bf16*)dnv_b, (bf16*)dphi, (bf16*)dpsi,
                       (bf16*)dv);
    hipLaunchKernelGGL(k_block_dsref<bf16>, pgrid, dim3(blk::kThreads), 0, s, bh, seq_len, d_k, d_v,
                       (const bf16*)phi, (const bf16*)dv, dsref_part);
  } else {
    hipLaunchKernelGGL(k_block_merge<float>, grid, dim3(blk::kThreads), smem, s, bh, seq_len, d_k, d_v, S_ref,
                       (const float*)dphi_b, (const float*)dpsi_b, (const float*)dnv_b, (float*)dphi, (float*)dpsi,
                       (float*)dv);
    hipLaunchKernelGGL(k_block_dsref<float>, pgrid, dim3(blk::kThreads), 0, s, bh, seq_len, d_k, d_v,
                       (const float*)phi, (const float*)dv, dsref_part);
  }
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

int atlas_replicas(int op, int dtype, int count, int nrep, const int64_t* n, const void* const* src,
                   void* const* dst, void* stream) {
  using namespace atlas;
  if (op != ATLAS_REPLICATE && op != ATLAS_REPLICA_SUM) return ATLAS_MEM_ERR_ARG;
  if (dtype != ATLAS_DT_F32 && dtype != ATLAS_DT_BF16) return ATLAS_MEM_ERR_DTYPE;
  if (count < 1 || count > rep::kMax || nrep < 1 || nrep > 64) return ATLAS_MEM_ERR_SHAPE;
  if (!n || !src || !dst) return ATLAS_MEM_ERR_NULL;
  rep::List L = {};
  L.count = count;
  L.nrep = nrep;
  const int esize = dtype == ATLAS_DT_BF16 ? 2 : 4;
  long total = 0;
  for (int z = 0; z < count; ++z) {
    if (n[z] < 0 || n[z] * nrep >= ((int64_t)1 << 40)) return ATLAS_MEM_ERR_SHAPE;
    if (n[z] > 0 && (!src[z] || !dst[z])) return ATLAS_MEM_ERR_NULL;
    if ((reinterpret_cast<uintptr_t>(src[z]) | reinterpret_cast<uintptr_t>(dst[z])) % esize) return ATLAS_MEM_ERR_ALIGN;
    L.src[z] = src[z];
    L.dst[z] = dst[z];
    L.n[z] = (long)n[z];
    L.vec[z] = n[z] % rep::kVec == 0 && !blk_misaligned(src[z]) && !blk_misaligned(dst[z]);
    L.off[z] = total;
    total += (n[z] + rep::kVec - 1) / rep::kVec;
  }
  L.off[count] = total;
  if (total == 0) return ATLAS_MEM_OK;
  if ((total + rep::kThreads - 1) / rep::kThreads >= ((int64_t)1 << 31)) return ATLAS_MEM_ERR_SHAPE;
  const dim3 grid((unsigned)((total + rep::kThreads - 1) / rep::kThreads));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == ATLAS_DT_BF16) {
    if (op == ATLAS_REPLICA_SUM) hipLaunchKernelGGL((atlas::k_replicas<bf16, true>), grid, dim3(rep::kThreads), 0, s, L);
    else hipLaunchKernelGGL((atlas::k_replicas<bf16, false>), grid, dim3(rep::kThreads), 0, s, L);
  } else {
    if (op == ATLAS_REPLICA_SUM) hipLaunchKernelGGL((atlas::k_replicas<float, true>), grid, dim3(rep::kThreads), 0, s, L);
    else hipLaunchKernelGGL((atlas::k_replicas<float, false>), grid, dim3(rep::kThreads), 0, s, L);
  }
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

}  // extern "C"
