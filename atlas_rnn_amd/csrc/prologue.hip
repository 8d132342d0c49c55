// prologue.hip - the memory cell's prologue around its projections (atlas_pytorch/rnn_memory.py:567-653,
// MultiheadRMSNorm :139-147), fused into two kernels on each side of the GEMMs (which stay on
// hipBLASLt):
//
//   k_pro_fwd   : xn = RMSNorm(x) (nn.RMSNorm(dim): x * rsqrt(mean(x^2) + eps) * w), and the three
//                 depthwise convolutions over time of xn (Conv1d(dim, dim, K, padding = K / 2,
//                 groups = dim, no bias), truncated to T: out[t] = sum_j w[c][j] xn[t + j - K/2], so
//                 for K = 4 token t sees t + 1) -> xn, q_in, k_in, v_in [B, T, dim]
//   (q_in, k_in, v_in, xn) @ (Wq, Wk, Wv, Wgates)^T on hipBLASLt
//   k_heads_fwd : per (b, t, h) row the head split to the recurrence's [(b h), T, d] layout,
//                 MultiheadRMSNorm of q and k (x / max(|x| d^-1/2, 1e-8) * gamma[h]), and the gate heads'
//                 bias + sigmoid -> q, k, v [(b h), T, d], gates [nG][(b h), T]
// and their adjoints k_heads_bwd / k_pro_bwd. Parameter gradients (norm weights, conv taps, gammas,
// gate biases) are written as per-workgroup partial sums that the host sums (deterministic).
//
// Workgroup = 256 threads over kTok tokens of one batch row and every channel; the per-token
// reductions (RMS over dim, the RMSNorm adjoint's dot product) go through LDS.
#include <hip/hip_runtime.h>

#include "../../include/atlas_mem.h"
#include "mem_common.h"

namespace atlas {

namespace pro {
constexpr int kThreads = 256;
constexpr int kTok = 16;        // tokens per workgroup
constexpr int kMaxK = 8;        // conv taps
constexpr int kHalo = kMaxK;    // halo tokens kept on each side (>= K)
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// inverse RMS of x[b, t, :] for t in [tb, te) into sinv[t - tb] (one wave per token).
template <typename T>
__device__ __forceinline__ void token_inv_rms(const T* xb, int dim, float eps, int tb, int te, float* sinv) {
  const int lane = lane_id(), w = wave_id();
  for (int t = tb + w; t < te; t += pro::kThreads / 64) {
    const T* row = xb + (size_t)t * dim;
    float s = 0.f;
    for (int c = lane; c < dim; c += 64) {
      const float v = to_f32(row[c]);
      s += v * v;
    }
    s = wave_sum(s);
    if (lane == 0) sinv[t - tb] = rsqrtf(s / (float)dim + eps);
  }
}

// Forward of RMSNorm + the three depthwise convolutions. wq / wk / wv: [dim][K] (null: no conv,
// then only xn is written). inv_rms [B][T] is saved for the backward.
template <typename T>
__global__ __launch_bounds__(pro::kThreads) void k_pro_fwd(int Tn, int dim, int K, int pad, float eps,
                                                           const T* __restrict__ x, const T* __restrict__ wn,
                                                           const T* __restrict__ wq, const T* __restrict__ wk,
                                                           const T* __restrict__ wv, T* __restrict__ xn,
                                                           T* __restrict__ qi, T* __restrict__ ki, T* __restrict__ vi,
                                                           float* __restrict__ inv_rms) {
  __shared__ float sinv[pro::kTok + 2 * pro::kHalo];
  const int t0 = blockIdx.x * pro::kTok, b = blockIdx.y, tid = threadIdx.x;
  const int t1 = min(Tn, t0 + pro::kTok);
  const bool conv = wq != nullptr;
  // tokens whose normalised values this tile reads: [t0 - pad, t1 - 1 + K - 1 - pad]
  const int hb = conv ? max(0, t0 - pad) : t0, he = conv ? min(Tn, t1 + K - 1 - pad) : t1;
  const int base = t0 - pro::kHalo;   // sinv index = t - base
  const T* xb = x + (size_t)b * Tn * dim;
  token_inv_rms(xb, dim, eps, hb, he, sinv + (hb - base));
  __syncthreads();
  for (int t = t0 + tid; t < t1; t += pro::kThreads) inv_rms[(size_t)b * Tn + t] = sinv[t - base];
  const size_t ob = (size_t)b * Tn * dim;
  for (int c = tid; c < dim; c += pro::kThreads) {
    const float w = to_f32(wn[c]);
    float tq[pro::kMaxK], tk[pro::kMaxK], tv[pro::kMaxK];
    if (conv) {
      for (int j = 0; j < K; ++j) {
        tq[j] = to_f32(wq[c * K + j]);
        tk[j] = to_f32(wk[c * K + j]);
        tv[j] = to_f32(wv[c * K + j]);
      }
    }
    for (int t = t0; t < t1; ++t) {
      xn[ob + (size_t)t * dim + c] = from_f32<T>(to_f32(xb[(size_t)t * dim + c]) * sinv[t - base] * w);
      if (!conv) continue;
      float aq = 0.f, ak = 0.f, av = 0.f;
      for (int j = 0; j < K; ++j) {
        const int s = t + j - pad;
        if (s < 0 || s >= Tn) continue;
        const float v = to_f32(xb[(size_t)s * dim + c]) * sinv[s - base] * w;
        aq += tq[j] * v;
        ak += tk[j] * v;
        av += tv[j] * v;
      }
      qi[ob + (size_t)t * dim + c] = from_f32<T>(aq);
      ki[ob + (size_t)t * dim + c] = from_f32<T>(ak);
      vi[ob + (size_t)t * dim + c] = from_f32<T>(av);
    }
  }
}

// Adjoint of k_pro_fwd. dxn: gradient reaching xn directly (the gate heads; with no conv also the
// projections); dqi / dki / dvi: gradients of the conv outputs (null without conv). Writes dx and
// per-workgroup partials dwn_part [nwg][dim], dwc_part [nwg][3][dim][K] (nwg = gridDim.x * gridDim.y).
//   u[t, c]  = w[c] * g[t, c],  g = dxn + sum_j taps[c][j] dconv[t - j + pad]   (the conv's transpose)
//   dx[t, c] = inv_t u[t, c] - x[t, c] inv_t^3 (sum_c' u[t, c'] x[t, c']) / dim
template <typename T>
__global__ __launch_bounds__(pro::kThreads) void k_pro_bwd(int Tn, int dim, int K, int pad, const T* __restrict__ x,
                                                           const T* __restrict__ wn, const T* __restrict__ wq,
                                                           const T* __restrict__ wk, const T* __restrict__ wv,
                                                           const float* __restrict__ inv_rms,
                                                           const T* __restrict__ dxn, const T* __restrict__ dqi,
                                                           const T* __restrict__ dki, const T* __restrict__ dvi,
                                                           T* __restrict__ dx, float* __restrict__ dwn_part,
                                                           float* __restrict__ dwc_part) {
  __shared__ float sdot[pro::kThreads / 64][pro::kTok];
  const int t0 = blockIdx.x * pro::kTok, b = blockIdx.y, tid = threadIdx.x, lane = lane_id(), wv_ = wave_id();
  const int t1 = min(Tn, t0 + pro::kTok), nt = t1 - t0;
  const int wg = blockIdx.y * gridDim.x + blockIdx.x;
  const bool conv = wq != nullptr;
  const size_t ob = (size_t)b * Tn * dim;
  const float* inv = inv_rms + (size_t)b * Tn;
  float dot[pro::kTok];
#pragma unroll
  for (int i = 0; i < pro::kTok; ++i) dot[i] = 0.f;
  // pass A: dot products, norm-weight and tap partials
  for (int c = tid; c < dim; c += pro::kThreads) {
    const float w = to_f32(wn[c]);
    float tq[pro::kMaxK], tk[pro::kMaxK], tv[pro::kMaxK], gq[pro::kMaxK], gk[pro::kMaxK], gv[pro::kMaxK];
    for (int j = 0; j < K; ++j) {
      tq[j] = conv ? to_f32(wq[c * K + j]) : 0.f;
      tk[j] = conv ? to_f32(wk[c * K + j]) : 0.f;
      tv[j] = conv ? to_f32(wv[c * K + j]) : 0.f;
      gq[j] = gk[j] = gv[j] = 0.f;
    }
    float dw = 0.f;
#pragma unroll
    for (int i = 0; i < pro::kTok; ++i) {
      const int t = t0 + i;
      if (t >= t1) break;
      const size_t o = ob + (size_t)t * dim + c;
      const float xv = to_f32(x[o]);
      float g = to_f32(dxn[o]);
      if (conv) {
        const float dq = to_f32(dqi[o]), dk = to_f32(dki[o]), dv = to_f32(dvi[o]);
        for (int j = 0; j < K; ++j) {
          // the conv's transpose: xn[t] feeds outputs u = t - j + pad
          const int u = t - j + pad;
          if (u >= 0 && u < Tn) {
            const size_t ou = ob + (size_t)u * dim + c;
            g += tq[j] * to_f32(dqi[ou]) + tk[j] * to_f32(dki[ou]) + tv[j] * to_f32(dvi[ou]);
          }
          // taps: output t reads xn[t + j - pad]
          const int s = t + j - pad;
          if (s >= 0 && s < Tn) {
            const float xs = to_f32(x[ob + (size_t)s * dim + c]) * inv[s] * w;
            gq[j] += dq * xs;
            gk[j] += dk * xs;
            gv[j] += dv * xs;
          }
        }
      }
      dw += g * xv * inv[t];
      dot[i] += w * g * xv;
    }
    dwn_part[(size_t)wg * dim + c] = dw;
    if (conv) {
      float* p = dwc_part + (size_t)wg * 3 * dim * K;
      for (int j = 0; j < K; ++j) {
        p[(size_t)c * K + j] = gq[j];
        p[(size_t)(dim + c) * K + j] = gk[j];
        p[(size_t)(2 * dim + c) * K + j] = gv[j];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < pro::kTok; ++i) {
    const float s = wave_sum(dot[i]);
    if (lane == 0) sdot[wv_][i] = s;
  }
  __syncthreads();
  // pass B: dx (recomputing u)
  for (int c = tid; c < dim; c += pro::kThreads) {
    const float w = to_f32(wn[c]);
    float tq[pro::kMaxK], tk[pro::kMaxK], tv[pro::kMaxK];
    for (int j = 0; j < K; ++j) {
      tq[j] = conv ? to_f32(wq[c * K + j]) : 0.f;
      tk[j] = conv ? to_f32(wk[c * K + j]) : 0.f;
      tv[j] = conv ? to_f32(wv[c * K + j]) : 0.f;
    }
    for (int i = 0; i < nt; ++i) {
      const int t = t0 + i;
      const size_t o = ob + (size_t)t * dim + c;
      float g = to_f32(dxn[o]);
      if (conv) {
        for (int j = 0; j < K; ++j) {
          const int u = t - j + pad;
          if (u >= 0 && u < Tn) {
            const size_t ou = ob + (size_t)u * dim + c;
            g += tq[j] * to_f32(dqi[ou]) + tk[j] * to_f32(dki[ou]) + tv[j] * to_f32(dvi[ou]);
          }
        }
      }
      const float it = inv[t];
      const float d = sdot[0][i] + sdot[1][i] + sdot[2][i] + sdot[3][i];
      dx[o] = from_f32<T>(it * w * g - to_f32(x[o]) * it * it * it * d / (float)dim);
    }
  }
}

// Head split + q / k MultiheadRMSNorm + gate sigmoids. ql, kl, vl [B, T, H d]; zl [B, T, nG H] gate
// logits (no bias); qg, kg [H][d] (null: no norm); bias [nG H]. Outputs q, k, v [(b h), T, d] and
// gates [nG][(b h), T]. One wave per (t, h) row of d <= 128 elements.
template <typename T>
__global__ __launch_bounds__(pro::kThreads) void k_heads_fwd(int Tn, int H, int d, int nG, const T* __restrict__ ql,
                                                             const T* __restrict__ kl, const T* __restrict__ vl,
                                                             const T* __restrict__ zl, const T* __restrict__ qg,
                                                             const T* __restrict__ kg, const T* __restrict__ bias,
                                                             T* __restrict__ q, T* __restrict__ k, T* __restrict__ v,
                                                             T* __restrict__ gates) {
  const int t0 = blockIdx.x * pro::kTok, b = blockIdx.y, tid = threadIdx.x, lane = lane_id(), w = wave_id();
  const int t1 = min(Tn, t0 + pro::kTok);
  const int HD = H * d, BH = gridDim.y * H;
  const float rs = rsqrtf((float)d);
  for (int r = w; r < (t1 - t0) * H; r += pro::kThreads / 64) {
    const int t = t0 + r / H, h = r % H;
    const size_t src = ((size_t)b * Tn + t) * HD + (size_t)h * d;
    const size_t dst = (((size_t)b * H + h) * Tn + t) * d;
    for (int which = 0; which < 3; ++which) {
      const T* in = which == 0 ? ql : (which == 1 ? kl : vl);
      T* out = which == 0 ? q : (which == 1 ? k : v);
      const T* gam = which == 0 ? qg : (which == 1 ? kg : nullptr);
      const float v0 = lane < d ? to_f32(in[src + lane]) : 0.f;
      const float v1 = lane + 64 < d ? to_f32(in[src + lane + 64]) : 0.f;
      float scale = 1.f;
      if (gam) {
        const float ss = wave_sum(v0 * v0 + v1 * v1);
        scale = 1.f / fmaxf(sqrtf(ss) * rs, 1e-8f);
      }
      if (lane < d) out[dst + lane] = from_f32<T>(v0 * scale * (gam ? to_f32(gam[h * d + lane]) : 1.f));
      if (lane + 64 < d) out[dst + lane + 64] = from_f32<T>(v1 * scale * (gam ? to_f32(gam[h * d + lane + 64]) : 1.f));
    }
  }
  // gates: one thread per (t, g, h)
  const int ng = (t1 - t0) * nG * H;
  for (int i = tid; i < ng; i += pro::kThreads) {
    const int t = t0 + i / (nG * H), gh = i % (nG * H), g = gh / H, h = gh % H;
    const float z = to_f32(zl[((size_t)b * Tn + t) * nG * H + gh]) + to_f32(bias[gh]);
    gates[((size_t)g * BH + (size_t)b * H + h) * Tn + t] = from_f32<T>(1.f / (1.f + __expf(-z)));
  }
}

// Adjoint of k_heads_fwd: dq, dk, dv [(b h), T, d], dgates [nG][(b h), T] (null: zero) and the forward's
// gates -> dql, dkl, dvl [B, T, H d], dzl [B, T, nG H]; partials dqg_part, dkg_part [nwg][H][d] (when
// the norms exist) and dbias_part [nwg][nG H].
//   y = x s gamma, s = 1 / max(r, 1e-8), r = |x| / sqrt(d):  dx = s gamma dy - x s^3 (x . gamma dy) / d  (r > 1e-8)
template <typename T>
__global__ __launch_bounds__(pro::kThreads) void k_heads_bwd(int Tn, int H, int d, int nG, const T* __restrict__ ql,
                                                             const T* __restrict__ kl, const T* __restrict__ qg,
                                                             const T* __restrict__ kg, const T* __restrict__ gates,
                                                             const T* __restrict__ dq, const T* __restrict__ dk,
                                                             const T* __restrict__ dv, const T* __restrict__ dgates,
                                                             T* __restrict__ dql, T* __restrict__ dkl,
                                                             T* __restrict__ dvl, T* __restrict__ dzl,
                                                             float* __restrict__ dqg_part, float* __restrict__ dkg_part,
                                                             float* __restrict__ dbias_part) {
  extern __shared__ float sgam[];   // [2][H][d] gamma partials of this workgroup, then [nG H] bias partials
  const int t0 = blockIdx.x * pro::kTok, b = blockIdx.y, tid = threadIdx.x, lane = lane_id(), w = wave_id();
  const int t1 = min(Tn, t0 + pro::kTok);
  const int HD = H * d, BH = gridDim.y * H;
  const int wg = blockIdx.y * gridDim.x + blockIdx.x;
  const float rs = rsqrtf((float)d);
  const bool norm = qg != nullptr;
  float* sb = sgam + 2 * HD;
  for (int i = tid; i < 2 * HD + nG * H; i += pro::kThreads) sgam[i] = 0.f;
  __syncthreads();
  for (int r = w; r < (t1 - t0) * H; r += pro::kThreads / 64) {
    const int t = t0 + r / H, h = r % H;
    const size_t xo = ((size_t)b * Tn + t) * HD + (size_t)h * d;
    const size_t yo = (((size_t)b * H + h) * Tn + t) * d;
    for (int which = 0; which < 3; ++which) {
      const T* dy = which == 0 ? dq : (which == 1 ? dk : dv);
      T* dxo = which == 0 ? dql : (which == 1 ? dkl : dvl);
      const float g0 = lane < d ? to_f32(dy[yo + lane]) : 0.f;
      const float g1 = lane + 64 < d ? to_f32(dy[yo + lane + 64]) : 0.f;
      if (which == 2 || !norm) {
        if (lane < d) dxo[xo + lane] = from_f32<T>(g0);
        if (lane + 64 < d) dxo[xo + lane + 64] = from_f32<T>(g1);
        continue;
      }
      const T* in = which == 0 ? ql : kl;
      const T* gam = which == 0 ? qg : kg;
      const float x0 = lane < d ? to_f32(in[xo + lane]) : 0.f;
      const float x1 = lane + 64 < d ? to_f32(in[xo + lane + 64]) : 0.f;
      const float gm0 = lane < d ? to_f32(gam[h * d + lane]) : 0.f;
      const float gm1 = lane + 64 < d ? to_f32(gam[h * d + lane + 64]) : 0.f;
      const float ss = wave_sum(x0 * x0 + x1 * x1);
      const float r_ = sqrtf(ss) * rs;
      const bool live = r_ > 1e-8f;
      const float s = 1.f / fmaxf(r_, 1e-8f);
      const float u0 = gm0 * g0, u1 = gm1 * g1;
      const float xu = wave_sum(x0 * u0 + x1 * u1);
      const float c3 = live ? s * s * s * xu / (float)d : 0.f;
      if (lane < d) dxo[xo + lane] = from_f32<T>(s * u0 - x0 * c3);
      if (lane + 64 < d) dxo[xo + lane + 64] = from_f32<T>(s * u1 - x1 * c3);
      float* sg = sgam + which * HD + h * d;
      if (lane < d) atomicAdd(&sg[lane], g0 * x0 * s);
      if (lane + 64 < d) atomicAdd(&sg[lane + 64], g1 * x1 * s);
    }
  }
  // gates: dz = dg s (1 - s)
  const int ng = (t1 - t0) * nG * H;
  for (int i = tid; i < ng; i += pro::kThreads) {
    const int t = t0 + i / (nG * H), gh = i % (nG * H), g = gh / H, h = gh % H;
    const size_t go = ((size_t)g * BH + (size_t)b * H + h) * Tn + t;
    const float s = to_f32(gates[go]);
    const float dg = dgates ? to_f32(dgates[go]) : 0.f;
    const float dz = dg * s * (1.f - s);
    dzl[((size_t)b * Tn + t) * nG * H + gh] = from_f32<T>(dz);
    atomicAdd(&sb[gh], dz);
  }
  __syncthreads();
  if (norm) {
    for (int i = tid; i < HD; i += pro::kThreads) {
      dqg_part[(size_t)wg * HD + i] = sgam[i];
      dkg_part[(size_t)wg * HD + i] = sgam[HD + i];
    }
  }
  for (int i = tid; i < nG * H; i += pro::kThreads) dbias_part[(size_t)wg * nG * H + i] = sb[i];
}

}  // namespace atlas

using namespace atlas;

namespace {
bool pro_shapes_ok(int B, int Tn, int dim, int K) {
  return B >= 1 && B <= 65535 && Tn >= 1 && dim >= 1 && dim <= (1 << 16) && K >= 0 && K <= pro::kMaxK;
}
bool heads_shapes_ok(int B, int Tn, int H, int d, int nG) {
  return B >= 1 && B <= 65535 && Tn >= 1 && H >= 1 && d >= 1 && d <= 128 && nG >= 0 && nG <= 8 &&
         (size_t)(2 * H * d + nG * H) * 4 <= 64 * 1024;
}
}  // namespace

extern "C" {

int atlas_prologue_num_workgroups(int batch, int seq_len) {
  if (batch < 1 || seq_len < 1) return 0;
  return batch * ((seq_len + pro::kTok - 1) / pro::kTok);
}

int atlas_prologue_fwd(int dtype, int batch, int seq_len, int dim, int conv_k, float eps, const void* x,
                       const void* norm_w, const void* wq, const void* wk, const void* wv, void* xn, void* q_in,
                       void* k_in, void* v_in, float* inv_rms, void* stream) {
  if (dtype != ATLAS_DT_F32 && dtype != ATLAS_DT_BF16) return ATLAS_MEM_ERR_DTYPE;
  if (!pro_shapes_ok(batch, seq_len, dim, conv_k)) return ATLAS_MEM_ERR_SHAPE;
  const bool conv = conv_k > 1;
  if (!x || !norm_w || !xn || !inv_rms) return ATLAS_MEM_ERR_NULL;
  if (conv && (!wq || !wk || !wv || !q_in || !k_in || !v_in)) return ATLAS_MEM_ERR_NULL;
  const dim3 grid((seq_len + pro::kTok - 1) / pro::kTok, batch);
  const int K = conv ? conv_k : 0, pad = conv_k / 2;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == ATLAS_DT_BF16)
    hipLaunchKernelGGL(k_pro_fwd<bf16>, grid, dim3(pro::kThreads), 0, s, seq_len, dim, K, pad, eps, (const bf16*)x,
                       (const bf16*)norm_w, conv ? (const bf16*)wq : nullptr, (const bf16*)wk, (const bf16*)wv,
                       (bf16*)xn, (bf16*)q_in, (bf16*)k_in, (bf16*)v_in, inv_rms);
  else
    hipLaunchKernelGGL(k_pro_fwd<float>, grid, dim3(pro::kThreads), 0, s, seq_len, dim, K, pad, eps, (const float*)x,
                       (const float*)norm_w, conv ? (const float*)wq : nullptr, (const float*)wk, (const float*)wv,
                       (float*)xn, (float*)q_in, (float*)k_in, (float*)v_in, inv_rms);
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

int atlas_prologue_bwd(int dtype, int batch, int seq_len, int dim, int conv_k, const void* x, const void* norm_w,
                       const void* wq, const void* wk, const void* wv, const float* inv_rms, const void* dxn,
                       const void* dq_in, const void* dk_in, const void* dv_in, void* dx, float* dnorm_w_part,
                       float* dconv_part, void* stream) {
  if (dtype != ATLAS_DT_F32 && dtype != ATLAS_DT_BF16) return ATLAS_MEM_ERR_DTYPE;
  if (!pro_shapes_ok(batch, seq_len, dim, conv_k)) return ATLAS_MEM_ERR_SHAPE;
  const bool conv = conv_k > 1;
  if (!x || !norm_w || !inv_rms || !dxn || !dx || !dnorm_w_part) return ATLAS_MEM_ERR_NULL;
  if (conv && (!wq || !wk || !wv || !dq_in || !dk_in || !dv_in || !dconv_part)) return ATLAS_MEM_ERR_NULL;
  const dim3 grid((seq_len + pro::kTok - 1) / pro::kTok, batch);
  const int K = conv ? conv_k : 0, pad = conv_k / 2;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == ATLAS_DT_BF16)
    hipLaunchKernelGGL(k_pro_bwd<bf16>, grid, dim3(pro::kThreads), 0, s, seq_len, dim, K, pad, (const bf16*)x,
                       (const bf16*)norm_w, conv ? (const bf16*)wq : nullptr, (const bf16*)wk, (const bf16*)wv, inv_rms,
                       (const bf16*)dxn, (const bf16*)dq_in, (const bf16*)dk_in, (const bf16*)dv_in, (bf16*)dx,
                       dnorm_w_part, dconv_part);
  else
    hipLaunchKernelGGL(k_pro_bwd<float>, grid, dim3(pro::kThreads), 0, s, seq_len, dim, K, pad, (const float*)x,
                       (const float*)norm_w, conv ? (const float*)wq : nullptr, (const float*)wk, (const float*)wv,
                       inv_rms, (const float*)dxn, (const float*)dq_in, (const float*)dk_in, (const float*)dv_in,
                       (float*)dx, dnorm_w_part, dconv_part);
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

int atlas_heads_fwd(int dtype, int batch, int seq_len, int heads, int d, int n_gates, const void* ql, const void* kl,
                    const void* vl, const void* zl, const void* q_gamma, const void* k_gamma, const void* gate_bias,
                    void* q, void* k, void* v, void* gates, void* stream) {
  if (dtype != ATLAS_DT_F32 && dtype != ATLAS_DT_BF16) return ATLAS_MEM_ERR_DTYPE;
  if (!heads_shapes_ok(batch, seq_len, heads, d, n_gates)) return ATLAS_MEM_ERR_SHAPE;
  if (!ql || !kl || !vl || !q || !k || !v) return ATLAS_MEM_ERR_NULL;
  if ((q_gamma == nullptr) != (k_gamma == nullptr)) return ATLAS_MEM_ERR_ARG;
  if (n_gates > 0 && (!zl || !gate_bias || !gates)) return ATLAS_MEM_ERR_NULL;
  const dim3 grid((seq_len + pro::kTok - 1) / pro::kTok, batch);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == ATLAS_DT_BF16)
    hipLaunchKernelGGL(k_heads_fwd<bf16>, grid, dim3(pro::kThreads), 0, s, seq_len, heads, d, n_gates, (const bf16*)ql,
                       (const bf16*)kl, (const bf16*)vl, (const bf16*)zl, (const bf16*)q_gamma, (const bf16*)k_gamma,
                       (const bf16*)gate_bias, (bf16*)q, (bf16*)k, (bf16*)v, (bf16*)gates);
  else
    hipLaunchKernelGGL(k_heads_fwd<float>, grid, dim3(pro::kThreads), 0, s, seq_len, heads, d, n_gates,
                       (const float*)ql, (const float*)kl, (const float*)vl, (const float*)zl, (const float*)q_gamma,
                       (const float*)k_gamma, (const float*)gate_bias, (float*)q, (float*)k, (float*)v, (float*)gates);
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

int atlas_heads_bwd(int dtype, int batch, int seq_len, int heads, int d, int n_gates, const void* ql, const void* kl,
                    const void* q_gamma, const void* k_gamma, const void* gates, const void* dq, const void* dk,
                    const void* dv, const void* dgates, void* dql, void* dkl, void* dvl, void* dzl,
                    float* dq_gamma_part, float* dk_gamma_part, float* dbias_part, void* stream) {
  if (dtype != ATLAS_DT_F32 && dtype != ATLAS_DT_BF16) return ATLAS_MEM_ERR_DTYPE;
  if (!heads_shapes_ok(batch, seq_len, heads, d, n_gates)) return ATLAS_MEM_ERR_SHAPE;
  if (!ql || !kl || !dq || !dk || !dv || !dql || !dkl || !dvl) return ATLAS_MEM_ERR_NULL;
  if ((q_gamma == nullptr) != (k_gamma == nullptr)) return ATLAS_MEM_ERR_ARG;
  if (q_gamma && (!dq_gamma_part || !dk_gamma_part)) return ATLAS_MEM_ERR_NULL;
  if (n_gates > 0 && (!gates || !dzl || !dbias_part)) return ATLAS_MEM_ERR_NULL;
  const dim3 grid((seq_len + pro::kTok - 1) / pro::kTok, batch);
  const size_t smem = (size_t)(2 * heads * d + n_gates * heads) * sizeof(float);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == ATLAS_DT_BF16)
    hipLaunchKernelGGL(k_heads_bwd<bf16>, grid, dim3(pro::kThreads), smem, s, seq_len, heads, d, n_gates,
                       (const bf16*)ql, (const bf16*)kl, (const bf16*)q_gamma, (const bf16*)k_gamma,
                       (const bf16*)gates, (const bf16*)dq, (const bf16*)dk, (const bf16*)dv, (const bf16*)dgates,
                       (bf16*)dql, (bf16*)dkl, (bf16*)dvl, (bf16*)dzl, dq_gamma_part, dk_gamma_part, dbias_part);
  else
    hipLaunchKernelGGL(k_heads_bwd<float>, grid, dim3(pro::kThreads), smem, s, seq_len, heads, d, n_gates,
                       (const float*)ql, (const float*)kl, (const float*)q_gamma, (const float*)k_gamma,
                       (const float*)gates, (const float*)dq, (const float*)dk, (const float*)dv, (const float*)dgates,
                       (float*)dql, (float*)dkl, (float*)dvl, (float*)dzl, dq_gamma_part, dk_gamma_part, dbias_part);
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

}  // extern "C"
