// affine.hip - right-affine scan H_t = H_{t-1} A_t + B_t (atlas_pytorch/affine_scan.py:36-158),
// chunked on the fp32 matrix cores (v_mfma_f32_16x16x4_f32).
//
// A: [N][T][D][D], B: [N][T][R][D], prev = H_0: [N][R][D] (zero when absent); out = H_1 .. H_T as
// [N][T][R][D]; fp32, D, R <= 64 (zero-padded to 64 x 64 operands inside LDS).
//
// The steps are cut into chunks of L; a chunk's steps compose to one affine map X -> X P_c + Q_c.
//   k_aff_compose : one workgroup per (n, chunk): P_c = prod of the chunk's matrices, Q_c = the
//                   chunk's scan from a zero start (L products of each kind, in parallel over chunks)
//   k_aff_chain   : one workgroup per n: the chunk-start states X_c, X_{c+1} = X_c P_c + Q_c
//   k_aff_apply   : one workgroup per (n, chunk): the chunk's steps from X_c, writing every H_t
// The scan's serial depth is L + T / L matrix products instead of T, and all but the chain run
// on N * T / L workgroups. Each step is one barrier: the step's matrix is double buffered in LDS
// and loaded one step ahead through registers, and the running state's rows are private to the
// wave that computes them.
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
constexpr int kMax = 64;        // D, R <= 64; every operand is zero-padded to 64 x 64 in LDS
constexpr int P = kMax + 1;     // LDS pitch (fp32)
constexpr int NE = kMax * kMax / kThreads;   // elements of a 64 x 64 operand per thread (16)
typedef MM<float> M;

struct Geo {
  int N, T, R, D, L, nc;
  int rev;   // 0: forward scan over A; 1: adjoint scan over A^T, backwards in time
};

// Scan step k (0 .. T-1) touches array position p: k forward, T-1-k in reverse.
__device__ __forceinline__ int pos(const Geo& g, int k) { return g.rev ? g.T - 1 - k : k; }

// A product C = X S on the matrix cores. Wave w owns the output rows 16 w .. 16 w + 15, all four
// 16-column tiles: acc[nt][r] = C[16 w + 4 kq + r][16 nt + tl] (tl = lane & 15, kq = lane >> 4). The
// k order is free as long as both operands follow it; lane group kq takes k = 16 kq + j at step j.
// XT / ST: X(m, k) = X[k][m] / S(k, n) = S[n][k] (the operand is stored transposed). With the pitch
// 65 every one of these scalar reads is free of bank conflicts in either orientation (the lanes of a
// read differ by tl + 16 kq + const modulo 64).
template <bool XT, bool ST>
__device__ __forceinline__ void prod(f32x4 (&acc)[4], const float (*X)[P], const float (*S)[P]) {
  const int l = lane_id(), w = wave_id(), tl = l & 15, kq = l >> 4;
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) acc[nt] = zero4();
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int k = 16 * kq + j;
    const float a = XT ? X[k][16 * w + tl] : X[16 * w + tl][k];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const float b = ST ? S[16 * nt + tl][k] : S[k][16 * nt + tl];
      acc[nt] = M::mma(a, b, acc[nt]);
    }
  }
}

// A rows x cols row-major matrix in memory (null: zeros; ident: the identity) through registers
// into a zero-padded 64 x 64 LDS operand, straight (s[r][c]) or transposed (s[c][r]). Thread t holds
// the 4-element groups t + 256 u (row (t + 256 u) / 16): coalesced loads (16-byte loads for a full
// 64 x 64 matrix), conflict-free LDS writes.
struct Pre {
  float v[NE];
};
__device__ __forceinline__ void pre_load(Pre& p, const float* src, int rows, int cols, bool ident = false) {
  const bool full = src && !ident && rows == kMax && cols == kMax;
#pragma unroll
  for (int u = 0; u < NE / 4; ++u) {
    const int v = threadIdx.x + kThreads * u, r = v / (kMax / 4), c = 4 * (v % (kMax / 4));
    if (full) {
      const float4 x = *reinterpret_cast<const float4*>(src + r * kMax + c);
      p.v[4 * u] = x.x; p.v[4 * u + 1] = x.y; p.v[4 * u + 2] = x.z; p.v[4 * u + 3] = x.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float x = 0.f;
        if (ident) x = r == c + i && r < rows ? 1.f : 0.f;
        else if (src && r < rows && c + i < cols) x = src[r * cols + c + i];
        p.v[4 * u + i] = x;
      }
    }
  }
}
template <bool T>
__device__ __forceinline__ void pre_store(const Pre& p, float (*s)[P]) {
#pragma unroll
  for (int u = 0; u < NE / 4; ++u) {
    const int v = threadIdx.x + kThreads * u, r = v / (kMax / 4), c = 4 * (v % (kMax / 4));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (T) s[c + i][r] = p.v[4 * u + i];
      else s[r][c + i] = p.v[4 * u + i];
    }
  }
}

// A rows x cols row-major matrix (null: zeros) in the accumulator layout of prod (16 per lane).
__device__ __forceinline__ void acc_load(float (&v)[16], const float* src, int rows, int cols) {
  const int l = lane_id(), w = wave_id(), tl = l & 15, kq = l >> 4;
  const bool full = src && rows == kMax && cols == kMax;
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * w + 4 * kq + r, col = 16 * nt + tl;
      v[4 * nt + r] = full ? src[row * kMax + col] : ((src && row < rows && col < cols) ? src[row * cols + col] : 0.f);
    }
}

// acc + add -> the wave's own rows of X (LDS) and, when out != null, memory (rows x cols).
__device__ __forceinline__ void acc_store(const f32x4 (&acc)[4], const float (&add)[16], float (*X)[P], float* out,
                                          int rows, int cols) {
  const int l = lane_id(), w = wave_id(), tl = l & 15, kq = l >> 4;
  const bool full = rows == kMax && cols == kMax;
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * w + 4 * kq + r, col = 16 * nt + tl;
      const float x = acc[nt][r] + add[4 * nt + r];
      X[row][col] = x;
      if (out && (full || (row < rows && col < cols))) out[row * cols + col] = x;
    }
}

// The step-k operand S_k: A[p] forward (used as stored), A[p + 1] in reverse (used transposed; the
// identity at k = 0, where nothing follows position T - 1).
__device__ __forceinline__ const float* step_mat(const Geo& g, const float* A, int n, int k) {
  const int p = pos(g, k);
  return A + ((size_t)n * g.T + (g.rev ? p + 1 : p)) * g.D * g.D;
}

}  // namespace aff

using aff::Geo;

// Rows of X and Pm are private to the wave that owns them (prod reads and acc_store writes only the
// wave's rows 16 w ..), so they need no barrier; the step operand S is shared and double buffered,
// loaded one step ahead through registers: one barrier per step.

// Phase 1: per (chunk c, n): P_c and Q_c of the chunk's steps k = c L .. min(T, c L + L) - 1.
// C = B (forward) or dout (reverse), indexed by array position.
template <bool REV>
__global__ __launch_bounds__(aff::kThreads) void k_aff_compose(Geo g, const float* __restrict__ A,
                                                               const float* __restrict__ C, float* __restrict__ Pc,
                                                               float* __restrict__ Qc) {
  __shared__ float S[2][aff::kMax][aff::P];
  __shared__ float X[aff::kMax][aff::P];    // running Q
  __shared__ float Pm[aff::kMax][aff::P];   // running product
  const int c = blockIdx.x, n = blockIdx.y, tid = threadIdx.x;
  const int k0 = c * g.L, k1 = min(g.T, k0 + g.L);
  const size_t cs = (size_t)g.R * g.D;
  aff::Pre ps;
  // step k0: P = S_k0, Q = C_k0
  aff::pre_load(ps, REV && k0 == 0 ? nullptr : aff::step_mat(g, A, n, k0), g.D, g.D, REV && k0 == 0);
  aff::pre_store<REV>(ps, Pm);
  aff::pre_load(ps, C + ((size_t)n * g.T + aff::pos(g, k0)) * cs, g.R, g.D);
  aff::pre_store<false>(ps, X);
  float cv[16];
  if (k0 + 1 < k1) {
    aff::pre_load(ps, aff::step_mat(g, A, n, k0 + 1), g.D, g.D);
    aff::pre_store<false>(ps, S[0]);
    aff::acc_load(cv, C + ((size_t)n * g.T + aff::pos(g, k0 + 1)) * cs, g.R, g.D);
    if (k0 + 2 < k1) aff::pre_load(ps, aff::step_mat(g, A, n, k0 + 2), g.D, g.D);
  }
  lds_barrier();
  for (int k = k0 + 1; k < k1; ++k) {
    const int b = (k - k0 - 1) & 1;
    f32x4 accP[4], accQ[4];
    aff::prod<false, REV>(accP, Pm, S[b]);
    aff::prod<false, REV>(accQ, X, S[b]);
    const float zero[16] = {};
    aff::acc_store(accP, zero, Pm, nullptr, 0, 0);
    aff::acc_store(accQ, cv, X, nullptr, 0, 0);
    if (k + 1 < k1) {
      aff::pre_store<false>(ps, S[b ^ 1]);
      aff::acc_load(cv, C + ((size_t)n * g.T + aff::pos(g, k + 1)) * cs, g.R, g.D);
      if (k + 2 < k1) aff::pre_load(ps, aff::step_mat(g, A, n, k + 2), g.D, g.D);
    }
    lds_barrier();
  }
  float* Pout = Pc + ((size_t)n * g.nc + c) * g.D * g.D;
  float* Qout = Qc + ((size_t)n * g.nc + c) * cs;
  for (int idx = tid; idx < g.D * g.D; idx += aff::kThreads) Pout[idx] = Pm[idx / g.D][idx % g.D];
  for (int idx = tid; idx < g.R * g.D; idx += aff::kThreads) Qout[idx] = X[idx / g.D][idx % g.D];
}

// Phase 2: per n, the start state of every chunk: X_0 = prev (forward) or 0 (reverse),
// X_{c+1} = X_c P_c + Q_c (P_c used as stored in either direction).
__global__ __launch_bounds__(aff::kThreads) void k_aff_chain(Geo g, const float* __restrict__ prev,
                                                             const float* __restrict__ Pc,
                                                             const float* __restrict__ Qc, float* __restrict__ Xc) {
  __shared__ float S[2][aff::kMax][aff::P];
  __shared__ float X[aff::kMax][aff::P];
  const int n = blockIdx.x;
  const size_t cs = (size_t)g.R * g.D;
  const float* pv = (!g.rev && prev) ? prev + (size_t)n * cs : nullptr;
  aff::Pre ps;
  aff::pre_load(ps, pv, g.R, g.D);
  aff::pre_store<false>(ps, X);
  {   // X_0 to memory (the element layout of pre_load)
    float* Xo = Xc + (size_t)n * g.nc * cs;
#pragma unroll
    for (int u = 0; u < aff::NE / 4; ++u) {
      const int v = threadIdx.x + aff::kThreads * u, r = v / (aff::kMax / 4), c4 = 4 * (v % (aff::kMax / 4));
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (r < g.R && c4 + i < g.D) Xo[r * g.D + c4 + i] = ps.v[4 * u + i];
    }
  }
  float qv[16];
  if (g.nc > 1) {
    aff::pre_load(ps, Pc + (size_t)n * g.nc * g.D * g.D, g.D, g.D);
    aff::pre_store<false>(ps, S[0]);
    aff::acc_load(qv, Qc + (size_t)n * g.nc * cs, g.R, g.D);
    if (g.nc > 2) aff::pre_load(ps, Pc + ((size_t)n * g.nc + 1) * g.D * g.D, g.D, g.D);
  }
  lds_barrier();
  for (int c = 0; c + 1 < g.nc; ++c) {
    const int b = c & 1;
    f32x4 acc[4];
    aff::prod<false, false>(acc, X, S[b]);
    aff::acc_store(acc, qv, X, Xc + ((size_t)n * g.nc + c + 1) * cs, g.R, g.D);
    if (c + 2 < g.nc) {
      aff::pre_store<false>(ps, S[b ^ 1]);
      aff::acc_load(qv, Qc + ((size_t)n * g.nc + c + 1) * cs, g.R, g.D);
      if (c + 3 < g.nc) aff::pre_load(ps, Pc + ((size_t)n * g.nc + c + 2) * g.D * g.D, g.D, g.D);
    }
    lds_barrier();
  }
}

// Phase 3: per (chunk c, n): the chunk's steps from X_c, every state written to out at its array
// position.
template <bool REV>
__global__ __launch_bounds__(aff::kThreads) void k_aff_apply(Geo g, const float* __restrict__ A,
                                                             const float* __restrict__ C,
                                                             const float* __restrict__ Xc, float* __restrict__ out) {
  __shared__ float S[2][aff::kMax][aff::P];
  __shared__ float X[aff::kMax][aff::P];
  const int c = blockIdx.x, n = blockIdx.y;
  const int k0 = c * g.L, k1 = min(g.T, k0 + g.L);
  const size_t cs = (size_t)g.R * g.D;
  aff::Pre ps;
  aff::pre_load(ps, Xc + ((size_t)n * g.nc + c) * cs, g.R, g.D);
  aff::pre_store<false>(ps, X);
  float cv[16];
  aff::pre_load(ps, REV && k0 == 0 ? nullptr : aff::step_mat(g, A, n, k0), g.D, g.D, REV && k0 == 0);
  aff::pre_store<false>(ps, S[0]);
  aff::acc_load(cv, C + ((size_t)n * g.T + aff::pos(g, k0)) * cs, g.R, g.D);
  if (k0 + 1 < k1) aff::pre_load(ps, aff::step_mat(g, A, n, k0 + 1), g.D, g.D);
  lds_barrier();
  for (int k = k0; k < k1; ++k) {
    const int b = (k - k0) & 1;
    f32x4 acc[4];
    aff::prod<false, REV>(acc, X, S[b]);
    aff::acc_store(acc, cv, X, out + ((size_t)n * g.T + aff::pos(g, k)) * cs, g.R, g.D);
    if (k + 1 < k1) {
      aff::pre_store<false>(ps, S[b ^ 1]);
      aff::acc_load(cv, C + ((size_t)n * g.T + aff::pos(g, k + 1)) * cs, g.R, g.D);
      if (k + 2 < k1) aff::pre_load(ps, aff::step_mat(g, A, n, k + 2), g.D, g.D);
    }
    lds_barrier();
  }
}

// dA_t = H_{t-1}^T G_t  (D x D, k over R) for every (t, n); workgroup t = T of each n forms
// dprev = G_1 A_1^T (R x D, k over D) when dprev is requested.
__global__ __launch_bounds__(aff::kThreads) void k_aff_grad_a(Geo g, const float* __restrict__ A,
                                                              const float* __restrict__ H,
                                                              const float* __restrict__ prev,
                                                              const float* __restrict__ G, float* __restrict__ dA,
                                                              float* __restrict__ dprev) {
  __shared__ float Xs[aff::kMax][aff::P];
  __shared__ float Ss[aff::kMax][aff::P];
  const int t = blockIdx.x, n = blockIdx.y;
  const size_t cs = (size_t)g.R * g.D;
  aff::Pre ps;
  const float zero[16] = {};
  f32x4 acc[4];
  if (t == g.T) {   // workgroup-uniform
    if (!dprev) return;
    // C[r][d] = sum_e G_1[r][e] A_1[d][e]: X = G_1 as stored, S(e, d) = A_1[d][e] (transposed)
    aff::pre_load(ps, G + (size_t)n * g.T * cs, g.R, g.D);
    aff::pre_store<false>(ps, Xs);
    aff::pre_load(ps, A + (size_t)n * g.T * g.D * g.D, g.D, g.D);
    aff::pre_store<false>(ps, Ss);
    __syncthreads();
    aff::prod<false, true>(acc, Xs, Ss);
    aff::acc_store(acc, zero, Xs, dprev + (size_t)n * cs, g.R, g.D);
    return;
  }
  // C[d][e] = sum_r H_{t-1}[r][d] G_t[r][e]: X(d, r) = H[r][d] (transposed), S(r, e) = G[r][e]
  const float* Hp = t > 0 ? H + ((size_t)n * g.T + t - 1) * cs : (prev ? prev + (size_t)n * cs : nullptr);
  aff::pre_load(ps, Hp, g.R, g.D);
  aff::pre_store<false>(ps, Xs);
  aff::pre_load(ps, G + ((size_t)n * g.T + t) * cs, g.R, g.D);
  aff::pre_store<false>(ps, Ss);
  __syncthreads();
  aff::prod<true, false>(acc, Xs, Ss);
  __syncthreads();   // every wave has read Xs before acc_store overwrites rows other waves read
  aff::acc_store(acc, zero, Xs, dA + ((size_t)n * g.T + t) * g.D * g.D, g.D, g.D);
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
  if (g.rev) hipLaunchKernelGGL(k_aff_compose<true>, dim3(g.nc, g.N), dim3(aff::kThreads), 0, s, g, A, C, Pc, Qc);
  else hipLaunchKernelGGL(k_aff_compose<false>, dim3(g.nc, g.N), dim3(aff::kThreads), 0, s, g, A, C, Pc, Qc);
  hipLaunchKernelGGL(k_aff_chain, dim3(g.N), dim3(aff::kThreads), 0, s, g, prev, Pc, Qc, Xc);
  if (g.rev) hipLaunchKernelGGL(k_aff_apply<true>, dim3(g.nc, g.N), dim3(aff::kThreads), 0, s, g, A, C, Xc, out);
  else hipLaunchKernelGGL(k_aff_apply<false>, dim3(g.nc, g.N), dim3(aff::kThreads), 0, s, g, A, C, Xc, out);
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
