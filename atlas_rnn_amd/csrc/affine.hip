// affine.hip - right-affine scan H_t = H_{t-1} A_t + B_t (atlas_pytorch/affine_scan.py:36-158),
// chunked on the fp32 matrix cores (v_mfma_f32_16x16x4_f32).
//
// A: [N][T][D][D], B: [N][T][R][D], prev = H_0: [N][R][D] (zero when absent); out = H_1 .. H_T as
// [N][T][R][D]; fp32, D, R <= 64 (padded to multiples of 16 inside LDS with zeros).
//
// The steps are cut into chunks of L; a chunk's steps compose to one affine map X -> X P_c + Q_c.
//   k_aff_compose : one workgroup per (n, chunk): P_c = prod of the chunk's matrices, Q_c = the
//                   chunk's scan from a zero start (L products of each kind, in parallel over chunks)
//   k_aff_chain   : one workgroup per n: the chunk-start states X_c, X_{c+1} = X_c P_c + Q_c
//   k_aff_apply   : one workgroup per (n, chunk): the chunk's steps from X_c, writing every H_t
// The scan's serial depth is L + T / L matrix products instead of T, and all but the chain run
// on N * T / L workgroups.
//
// Backward: with the adjoint G_t = dL/dH_t,  G_T = dout_T,  G_t = dout_t + G_{t+1} A_{t+1}^T, so G is the
// same scan run backwards in time over the transposed matrices (the `rev` mode of the three kernels,
// written straight into dB = G). Then k_aff_grad_a forms dA_t = H_{t-1}^T G_t for every (n, t) and
// dprev = G_1 A_1^T (one extra workgroup per n).
#include <hip/hip_runtime.h>

#include "../../include/atlas_mem.h"
#include "mem_common.h"

namespace atlas {

namespace aff {
constexpr int kThreads = 256;   // 4 waves
constexpr int kMax = 64;        // D, R <= 64
constexpr int P = kMax + 1;     // LDS pitch (fp32): column reads without bank conflicts
typedef MM<float> M;

struct Geo {
  int N, T, R, D, L, nc, RP, DP;   // RP / DP: R and D rounded up to 16
  int rev;                         // 0: forward scan over A; 1: adjoint scan over A^T, backwards in time
};

// Scan step k (0 .. T-1) touches array position p: k forward, T-1-k in reverse.
__device__ __forceinline__ int pos(const Geo& g, int k) { return g.rev ? g.T - 1 - k : k; }

// Stage the step-k matrix into s (row-major [d][e], zero padded to DP x DP): A[p] forward; in
// reverse A[p+1]^T, the identity for the first step (k = 0: nothing follows position T-1).
__device__ __forceinline__ void stage_mat(const Geo& g, const float* A, int n, int k, float (*s)[P]) {
  const int tid = threadIdx.x;
  const int p = pos(g, k);
  const bool ident = g.rev && k == 0;
  const float* src = ident ? nullptr : A + ((size_t)n * g.T + (g.rev ? p + 1 : p)) * g.D * g.D;
  for (int idx = tid; idx < g.DP * g.DP; idx += kThreads) {
    const int d = idx / g.DP, e = idx % g.DP;
    float v = 0.f;
    if (d < g.D && e < g.D) v = ident ? (d == e ? 1.f : 0.f) : (g.rev ? src[e * g.D + d] : src[d * g.D + e]);
    s[d][e] = v;
  }
}

// acc[j] += X (rows 16 mt.., k over DP) times S (k rows, columns 16 nt..) for the tiles this wave owns.
// Tile j of the wave is tile index w + 4 j of the (rows / 16) x (DP / 16) grid.
template <int NT>
__device__ __forceinline__ void mul_tiles(f32x4 (&acc)[NT], const float (*X)[P], const float (*S)[P], int rows,
                                          int DP) {
  const int l = lane_id(), w = wave_id();
  const int ct = DP / 16, ntile = (rows / 16) * ct;
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int t = w + 4 * j;
    const int tt = t < ntile ? t : 0;   // out-of-range tiles compute tile 0 and are not stored
    const int m0 = 16 * (tt / ct), n0 = 16 * (tt % ct);
    f32x4 a = zero4();
    for (int k0 = 0; k0 < DP; k0 += 4) a = M::mma(X[m0 + (l & 15)][k0 + (l >> 4)], S[k0 + (l >> 4)][n0 + (l & 15)], a);
    acc[j] = a;
  }
}

// Adds the step's input C (rows x D, global, row-major [r][e]) to acc and stores to Y (LDS) and,
// when out != null, to out (global). Padded rows / columns store zeros in Y.
template <int NT>
__device__ __forceinline__ void finish_tiles(const f32x4 (&acc)[NT], const float* C, float (*Y)[P], float* out,
                                             int rows, int rows_real, int D, int DP) {
  const int l = lane_id(), w = wave_id();
  const int ct = DP / 16, ntile = (rows / 16) * ct;
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int t = w + 4 * j;
    if (t >= ntile) continue;
    const int m0 = 16 * (t / ct), n0 = 16 * (t % ct);
    const int e = n0 + (l & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = m0 + 4 * (l >> 4) + i;
      const bool real = r < rows_real && e < D;
      float v = acc[j][i];
      if (C && real) v += C[r * D + e];
      v = real ? v : 0.f;
      Y[r][e] = v;
      if (out && real) out[r * D + e] = v;
    }
  }
}

struct Smem {
  float X[kMax][P];   // running state (R x D) or, in compose, the running Q
  float Pm[kMax][P];  // compose: running product (D x D)
  float S[kMax][P];   // the step's matrix
};

// tiles per wave: (64 / 16)^2 = 16 tiles over 4 waves
constexpr int NTW = 4;

}  // namespace aff

using aff::Geo;
using aff::Smem;

// Phase 1: per (chunk c, n): P_c and Q_c of the chunk's steps k = c L .. min(T, c L + L) - 1.
// C = B (forward) or dout (reverse), indexed by array position.
__global__ __launch_bounds__(aff::kThreads) void k_aff_compose(Geo g, const float* __restrict__ A,
                                                               const float* __restrict__ C, float* __restrict__ Pc,
                                                               float* __restrict__ Qc) {
  __shared__ Smem sm;
  const int c = blockIdx.x, n = blockIdx.y, tid = threadIdx.x;
  const int k0 = c * g.L, k1 = min(g.T, k0 + g.L);
  // step k0: P = its matrix, Q = its input
  aff::stage_mat(g, A, n, k0, sm.Pm);
  {
    const float* Ck = C + ((size_t)n * g.T + aff::pos(g, k0)) * g.R * g.D;
    for (int idx = tid; idx < g.RP * g.DP; idx += aff::kThreads) {
      const int r = idx / g.DP, e = idx % g.DP;
      sm.X[r][e] = (r < g.R && e < g.D) ? Ck[r * g.D + e] : 0.f;
    }
  }
  for (int k = k0 + 1; k < k1; ++k) {
    aff::stage_mat(g, A, n, k, sm.S);
    __syncthreads();
    f32x4 accP[aff::NTW], accQ[aff::NTW];
    aff::mul_tiles(accP, sm.Pm, sm.S, g.DP, g.DP);
    aff::mul_tiles(accQ, sm.X, sm.S, g.RP, g.DP);
    __syncthreads();
    const float* Ck = C + ((size_t)n * g.T + aff::pos(g, k)) * g.R * g.D;
    aff::finish_tiles(accP, nullptr, sm.Pm, nullptr, g.DP, g.D, g.D, g.DP);
    aff::finish_tiles(accQ, Ck, sm.X, nullptr, g.RP, g.R, g.D, g.DP);
  }
  __syncthreads();
  float* Pout = Pc + ((size_t)n * g.nc + c) * g.D * g.D;
  float* Qout = Qc + ((size_t)n * g.nc + c) * g.R * g.D;
  for (int idx = tid; idx < g.D * g.D; idx += aff::kThreads) Pout[idx] = sm.Pm[idx / g.D][idx % g.D];
  for (int idx = tid; idx < g.R * g.D; idx += aff::kThreads) Qout[idx] = sm.X[idx / g.D][idx % g.D];
}

// Phase 2: per n, the start state of every chunk: X_0 = prev (forward) or 0 (reverse),
// X_{c+1} = X_c P_c + Q_c.
__global__ __launch_bounds__(aff::kThreads) void k_aff_chain(Geo g, const float* __restrict__ prev,
                                                             const float* __restrict__ Pc,
                                                             const float* __restrict__ Qc, float* __restrict__ Xc) {
  __shared__ Smem sm;
  const int n = blockIdx.x, tid = threadIdx.x;
  const float* pv = (!g.rev && prev) ? prev + (size_t)n * g.R * g.D : nullptr;
  for (int idx = tid; idx < g.RP * g.DP; idx += aff::kThreads) {
    const int r = idx / g.DP, e = idx % g.DP;
    sm.X[r][e] = (pv && r < g.R && e < g.D) ? pv[r * g.D + e] : 0.f;
  }
  for (int c = 0; c < g.nc; ++c) {
    const float* Pm = Pc + ((size_t)n * g.nc + c) * g.D * g.D;
    for (int idx = tid; idx < g.DP * g.DP; idx += aff::kThreads) {
      const int d = idx / g.DP, e = idx % g.DP;
      sm.S[d][e] = (d < g.D && e < g.D) ? Pm[d * g.D + e] : 0.f;
    }
    __syncthreads();
    float* Xo = Xc + ((size_t)n * g.nc + c) * g.R * g.D;
    for (int idx = tid; idx < g.R * g.D; idx += aff::kThreads) Xo[idx] = sm.X[idx / g.D][idx % g.D];
    if (c + 1 == g.nc) break;
    f32x4 acc[aff::NTW];
    aff::mul_tiles(acc, sm.X, sm.S, g.RP, g.DP);
    __syncthreads();
    aff::finish_tiles(acc, Qc + ((size_t)n * g.nc + c) * g.R * g.D, sm.X, nullptr, g.RP, g.R, g.D, g.DP);
  }
}

// Phase 3: per (chunk c, n): the chunk's steps from X_c, every state written to out at its array
// position.
__global__ __launch_bounds__(aff::kThreads) void k_aff_apply(Geo g, const float* __restrict__ A,
                                                             const float* __restrict__ C,
                                                             const float* __restrict__ Xc, float* __restrict__ out) {
  __shared__ Smem sm;
  const int c = blockIdx.x, n = blockIdx.y, tid = threadIdx.x;
  const int k0 = c * g.L, k1 = min(g.T, k0 + g.L);
  const float* X0 = Xc + ((size_t)n * g.nc + c) * g.R * g.D;
  for (int idx = tid; idx < g.RP * g.DP; idx += aff::kThreads) {
    const int r = idx / g.DP, e = idx % g.DP;
    sm.X[r][e] = (r < g.R && e < g.D) ? X0[r * g.D + e] : 0.f;
  }
  for (int k = k0; k < k1; ++k) {
    aff::stage_mat(g, A, n, k, sm.S);
    __syncthreads();
    f32x4 acc[aff::NTW];
    aff::mul_tiles(acc, sm.X, sm.S, g.RP, g.DP);
    __syncthreads();
    const size_t off = ((size_t)n * g.T + aff::pos(g, k)) * g.R * g.D;
    aff::finish_tiles(acc, C + off, sm.X, out + off, g.RP, g.R, g.D, g.DP);
  }
}

// dA_t = H_{t-1}^T G_t  (D x D, k over R) for every (t, n); workgroup t = T of each n forms
// dprev = G_1 A_1^T (R x D, k over D) when dprev is requested.
__global__ __launch_bounds__(aff::kThreads) void k_aff_grad_a(Geo g, const float* __restrict__ A,
                                                              const float* __restrict__ H,
                                                              const float* __restrict__ prev,
                                                              const float* __restrict__ G, float* __restrict__ dA,
                                                              float* __restrict__ dprev) {
  __shared__ Smem sm;
  const int t = blockIdx.x, n = blockIdx.y, tid = threadIdx.x;
  if (t == g.T) {
    if (!dprev) return;
    // X = G_1 (R x D), S[e][d] = A_1[d][e] (A_1^T), dprev = X S
    const float* G1 = G + (size_t)n * g.T * g.R * g.D;
    const float* A1 = A + (size_t)n * g.T * g.D * g.D;
    for (int idx = tid; idx < g.RP * g.DP; idx += aff::kThreads) {
      const int r = idx / g.DP, e = idx % g.DP;
      sm.X[r][e] = (r < g.R && e < g.D) ? G1[r * g.D + e] : 0.f;
    }
    for (int idx = tid; idx < g.DP * g.DP; idx += aff::kThreads) {
      const int e = idx / g.DP, d = idx % g.DP;
      sm.S[e][d] = (e < g.D && d < g.D) ? A1[d * g.D + e] : 0.f;
    }
    __syncthreads();
    f32x4 acc[aff::NTW];
    aff::mul_tiles(acc, sm.X, sm.S, g.RP, g.DP);
    __syncthreads();
    aff::finish_tiles(acc, nullptr, sm.Pm, dprev + (size_t)n * g.R * g.D, g.RP, g.R, g.D, g.DP);
    return;
  }
  // X[d][r] = H_{t-1}[r][d] (D x RP), S[r][e] = G_t[r][e] (RP x D): dA_t = X S, k over RP
  const float* Hp = t > 0 ? H + ((size_t)n * g.T + t - 1) * g.R * g.D : (prev ? prev + (size_t)n * g.R * g.D : nullptr);
  const float* Gt = G + ((size_t)n * g.T + t) * g.R * g.D;
  for (int idx = tid; idx < g.DP * g.RP; idx += aff::kThreads) {
    const int d = idx / g.RP, r = idx % g.RP;
    sm.X[d][r] = (Hp && d < g.D && r < g.R) ? Hp[r * g.D + d] : 0.f;
  }
  for (int idx = tid; idx < g.RP * g.DP; idx += aff::kThreads) {
    const int r = idx / g.DP, e = idx % g.DP;
    sm.S[r][e] = (r < g.R && e < g.D) ? Gt[r * g.D + e] : 0.f;
  }
  __syncthreads();
  // rows d over DP, k over RP, columns e over DP
  const int l = lane_id(), w = wave_id();
  const int ct = g.DP / 16, ntile = ct * ct;
  float* dAt = dA + ((size_t)n * g.T + t) * g.D * g.D;
#pragma unroll
  for (int j = 0; j < aff::NTW; ++j) {
    const int tt = w + 4 * j;
    const int ts = tt < ntile ? tt : 0;
    const int m0 = 16 * (ts / ct), n0 = 16 * (ts % ct);
    f32x4 a = zero4();
    for (int k0 = 0; k0 < g.RP; k0 += 4)
      a = aff::M::mma(sm.X[m0 + (l & 15)][k0 + (l >> 4)], sm.S[k0 + (l >> 4)][n0 + (l & 15)], a);
    if (tt < ntile) {
      const int e = n0 + (l & 15);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = m0 + 4 * (l >> 4) + i;
        if (d < g.D && e < g.D) dAt[d * g.D + e] = a[i];
      }
    }
  }
}

}  // namespace atlas

using namespace atlas;

namespace {

int affine_check(int n, int t, int r, int d) {
  if (n < 1 || t < 1 || r < 1 || d < 1 || r > aff::kMax || d > aff::kMax) return ATLAS_MEM_ERR_SHAPE;
  return ATLAS_MEM_OK;
}

// Chunk length: about sqrt(2 T) steps (the compose pass runs L steps of two products, the chain
// T / L steps of one), a power of two in [4, 64].
int affine_chunk(int t) {
  int L = 4;
  while (L < 64 && (size_t)L * L < (size_t)2 * t) L *= 2;
  return L;
}

Geo affine_geo(int n, int t, int r, int d, int rev) {
  Geo g{};
  g.N = n; g.T = t; g.R = r; g.D = d;
  g.L = affine_chunk(t);
  g.nc = (t + g.L - 1) / g.L;
  g.RP = (r + 15) / 16 * 16;
  g.DP = (d + 15) / 16 * 16;
  g.rev = rev;
  return g;
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// workspace: P_c [N][nc][D][D], Q_c and X_c [N][nc][R][D]
size_t affine_ws_bytes(const Geo& g) {
  const size_t nc = (size_t)g.N * g.nc;
  return align256(nc * g.D * g.D * 4) + 2 * align256(nc * g.R * g.D * 4);
}

int affine_scan(const Geo& g, const float* A, const float* C, const float* prev, float* out, void* ws,
                hipStream_t s) {
  unsigned char* w = static_cast<unsigned char*>(ws);
  const size_t nc = (size_t)g.N * g.nc;
  float* Pc = reinterpret_cast<float*>(w);
  float* Qc = reinterpret_cast<float*>(w + align256(nc * g.D * g.D * 4));
  float* Xc = reinterpret_cast<float*>(w + align256(nc * g.D * g.D * 4) + align256(nc * g.R * g.D * 4));
  hipLaunchKernelGGL(k_aff_compose, dim3(g.nc, g.N), dim3(aff::kThreads), 0, s, g, A, C, Pc, Qc);
  hipLaunchKernelGGL(k_aff_chain, dim3(g.N), dim3(aff::kThreads), 0, s, g, prev, Pc, Qc, Xc);
  hipLaunchKernelGGL(k_aff_apply, dim3(g.nc, g.N), dim3(aff::kThreads), 0, s, g, A, C, Xc, out);
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

bool aff_misaligned(const void* p) { return p && (reinterpret_cast<uintptr_t>(p) & 3) != 0; }

}  // namespace

extern "C" {

size_t atlas_affine_scan_workspace_bytes(int n, int t, int r, int d) {
  if (affine_check(n, t, r, d) != ATLAS_MEM_OK) return 0;
  return affine_ws_bytes(affine_geo(n, t, r, d, 0));
}

int atlas_affine_scan_fwd(int n, int t, int r, int d, const float* A, const float* B, const float* prev, float* out,
                          void* workspace, size_t workspace_bytes, void* stream) {
  const int st = affine_check(n, t, r, d);
  if (st != ATLAS_MEM_OK) return st;
  if (!A || !B || !out || !workspace) return ATLAS_MEM_ERR_NULL;
  if (aff_misaligned(A) || aff_misaligned(B) || aff_misaligned(prev) || aff_misaligned(out) ||
      aff_misaligned(workspace))
    return ATLAS_MEM_ERR_ALIGN;
  const Geo g = affine_geo(n, t, r, d, 0);
  if (workspace_bytes < affine_ws_bytes(g)) return ATLAS_MEM_ERR_WORKSPACE;
  return affine_scan(g, A, B, prev, out, workspace, static_cast<hipStream_t>(stream));
}

int atlas_affine_scan_bwd(int n, int t, int r, int d, const float* A, const float* H, const float* prev,
                          const float* dout, float* dA, float* dB, float* dprev, void* workspace,
                          size_t workspace_bytes, void* stream) {
  const int st = affine_check(n, t, r, d);
  if (st != ATLAS_MEM_OK) return st;
  if (!A || !H || !dout || !dA || !dB || !workspace) return ATLAS_MEM_ERR_NULL;
  if (aff_misaligned(A) || aff_misaligned(H) || aff_misaligned(prev) || aff_misaligned(dout) || aff_misaligned(dA) ||
      aff_misaligned(dB) || aff_misaligned(dprev) || aff_misaligned(workspace))
    return ATLAS_MEM_ERR_ALIGN;
  const Geo g = affine_geo(n, t, r, d, 1);
  if (workspace_bytes < affine_ws_bytes(g)) return ATLAS_MEM_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // G (the adjoint of every H_t) is the reverse scan of dout over A^T; dB = G
  const int rc = affine_scan(g, A, dout, nullptr, dB, workspace, s);
  if (rc != ATLAS_MEM_OK) return rc;
  hipLaunchKernelGGL(k_aff_grad_a, dim3(t + 1, n), dim3(aff::kThreads), 0, s, g, A, H, prev, dB, dA, dprev);
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

}  // extern "C"
