// prologue.hip - the memory cell's prologue around its projections (atlas_pytorch/rnn_memory.py:567-653,
// MultiheadRMSNorm :139-147), fused into two kernels on each side of the products (gemm.hip,
// weight gradients wgrad.hip):
//
//   k_pro_fwd   : xn = RMSNorm(x) (nn.RMSNorm(dim): x * rsqrt(mean(x^2) + eps) * w), and the three
//                 depthwise convolutions over time of xn (Conv1d(dim, dim, K, padding = K / 2,
//                 groups = dim, no bias), truncated to T: out[t] = sum_j w[c][j] xn[t + j - K/2], so
//                 for K = 4 token t sees t + 1) -> xn, q_in, k_in, v_in [B, T, dim]
//   (q_in, k_in, v_in, xn) @ (Wq, Wk, Wv, Wgates)^T as one batched launch (gemm.hip)
//   k_heads_fwd : per (b, t, h) row the head split to the recurrence's [(b h), T, d] layout,
//                 MultiheadRMSNorm of q and k (x / max(|x| d^-1/2, 1e-8) * gamma[h]), and the gate heads'
//                 bias + sigmoid -> q, k, v [(b h), T, d], gates [nG][(b h), T]
// and their adjoints k_heads_bwd / k_pro_bwd. Parameter gradients (norm weights, conv taps, gammas,
// gate biases) are written as per-workgroup partial sums that the host sums (deterministic).
//
// Workgroup = 256 threads over kTok tokens of one batch row and every channel; the per-token
// reductions (RMS over dim, the RMSNorm adjoint's dot product) go through LDS.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "../../include/atlas_mem.h"
#include "mem_common.h"
#include "walk_common.h"

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

// inverse RMS of x[b, t, :] for t in [tb, te) into sinv[t - tb]: one wave per token, eight channels
// (one 16-byte vector of bf16) per lane.
template <typename T>
__device__ __forceinline__ void token_inv_rms(const T* xb, int dim, float eps, int tb, int te, float* sinv) {
  const int lane = lane_id(), w = wave_id();
  for (int t = tb + w; t < te; t += pro::kThreads / 64) {
    const T* row = xb + (size_t)t * dim;
    float s = 0.f;
    for (int c8 = lane * 8; c8 < dim; c8 += 512) {
      float v[8];
      ld8(row + c8, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) s += v[e] * v[e];
    }
    s = wave_sum(s);
    if (lane == 0) sinv[t - tb] = rsqrtf(s / (float)dim + eps);
  }
}

// the K taps of eight channels c8 .. c8 + 7 of a [dim][K] tap array, as tap[j][e]
template <typename T, int KT>
__device__ __forceinline__ void load_taps(const T* w, int c8, float (&tap)[KT > 0 ? KT : 1][8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int j = 0; j < KT; ++j) tap[j][e] = to_f32(w[(size_t)(c8 + e) * KT + j]);
}

// Forward of RMSNorm + the three depthwise convolutions (KT taps, 0: no conv, then only xn is
// written). inv_rms [B][T] is saved for the backward. Workgroup: 16 tokens of one batch row; lane l
// of wave w handles channels 8 l .. (every 512 channels) of tokens w, w + 4, ... with 16-byte accesses.
template <typename T, int KT>
__global__ __launch_bounds__(pro::kThreads) void k_pro_fwd(int Tn, int dim, float eps, const T* __restrict__ x,
                                                           const T* __restrict__ wn, const T* __restrict__ wq,
                                                           const T* __restrict__ wk, const T* __restrict__ wv,
                                                           T* __restrict__ xn, T* __restrict__ qi,
                                                           T* __restrict__ ki, T* __restrict__ vi,
                                                           float* __restrict__ inv_rms) {
  constexpr int pad = KT / 2;
  __shared__ float sinv[pro::kTok + 2 * pro::kHalo];
  const int t0 = blockIdx.x * pro::kTok, b = blockIdx.y, tid = threadIdx.x, lane = lane_id(), w = wave_id();
  const int t1 = min(Tn, t0 + pro::kTok);
  // tokens whose normalised values this tile reads: [t0 - pad, t1 - 1 + K - 1 - pad]
  const int hb = KT ? max(0, t0 - pad) : t0, he = KT ? min(Tn, t1 + KT - 1 - pad) : t1;
  const int base = t0 - pro::kHalo;   // sinv index = t - base
  const T* xb = x + (size_t)b * Tn * dim;
  token_inv_rms(xb, dim, eps, hb, he, sinv + (hb - base));
  __syncthreads();
  for (int t = t0 + tid; t < t1; t += pro::kThreads) inv_rms[(size_t)b * Tn + t] = sinv[t - base];
  const size_t ob = (size_t)b * Tn * dim;
  for (int c8 = lane * 8; c8 < dim; c8 += 512) {
    float wv8[8];
    ld8(wn + c8, wv8);
    float tq[KT > 0 ? KT : 1][8], tk[KT > 0 ? KT : 1][8], tv[KT > 0 ? KT : 1][8];
    if constexpr (KT > 0) {
      load_taps<T, KT>(wq, c8, tq);
      load_taps<T, KT>(wk, c8, tk);
      load_taps<T, KT>(wv, c8, tv);
    }
    for (int t = t0 + w; t < t1; t += pro::kThreads / 64) {
      float xv[8];
      ld8(xb + (size_t)t * dim + c8, xv);
      const float it = sinv[t - base];
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[e] *= it * wv8[e];
      st8(xn + ob + (size_t)t * dim + c8, xv);
      if constexpr (KT > 0) {
        float aq[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, ak[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f},
              av[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < KT; ++j) {
          const int s = t + j - pad;
          if (s < 0 || s >= Tn) continue;
          float xs[8];
          ld8(xb + (size_t)s * dim + c8, xs);
          const float is = sinv[s - base];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float v = xs[e] * is * wv8[e];
            aq[e] += tq[j][e] * v;
            ak[e] += tk[j][e] * v;
            av[e] += tv[j][e] * v;
          }
        }
        st8(qi + ob + (size_t)t * dim + c8, aq);
        st8(ki + ob + (size_t)t * dim + c8, ak);
        st8(vi + ob + (size_t)t * dim + c8, av);
      }
    }
  }
}

// Adjoint of k_pro_fwd. dxn: gradient reaching xn directly (the gate heads; with no conv also the
// projections); dqi / dki / dvi: gradients of the conv outputs (null without conv). Writes dx and
// partials dwn_part [nwg][dim], dwc_part [nwg][3][dim][K], nwg = B * ceil(T / 16): one workgroup per
// 16-token block of one batch row (partial row b * ceil(T / 16) + block); wave w owns tokens
// 4 w .. 4 w + 3 of the block and every channel, eight per lane.
//   u[t, c]  = w[c] * g[t, c],  g = dxn + sum_j taps[c][j] dconv[t - j + pad]   (the conv's transpose)
//   dx[t, c] = inv_t u[t, c] - x[t, c] inv_t^3 (sum_c' u[t, c'] x[t, c']) / dim
// Three passes: A (g: the dot products and the norm-weight partials), B (g again: dx), C (the tap
// partials), so that taps and tap partials are never live together; the four waves' partials are
// summed through LDS, 512 channels at a time.
template <typename T, int KT>
__global__ __launch_bounds__(pro::kThreads) void k_pro_bwd(int Tn, int dim, const T* __restrict__ x,
                                                           const T* __restrict__ wn, const T* __restrict__ wq,
                                                           const T* __restrict__ wk, const T* __restrict__ wv,
                                                           const float* __restrict__ inv_rms,
                                                           const T* __restrict__ dxn, const T* __restrict__ dqi,
                                                           const T* __restrict__ dki, const T* __restrict__ dvi,
                                                           T* __restrict__ dx, float* __restrict__ dwn_part,
                                                           float* __restrict__ dwc_part) {
  constexpr int pad = KT / 2, KA = KT > 0 ? KT : 1, NW = pro::kThreads / 64, TW = pro::kTok / NW;
  __shared__ float sred[NW][512 * KA];   // per-wave partials of 512 channels (x K taps)
  const int lane = lane_id(), w = wave_id(), tid = threadIdx.x;
  const int b = blockIdx.y, ntb = gridDim.x, blk = blockIdx.x;
  const int t0 = blk * pro::kTok + w * TW, t1 = min(Tn, t0 + TW);   // this wave's tokens (may be none)
  const size_t ob = (size_t)b * Tn * dim, prow = (size_t)b * ntb + blk;
  const float* inv = inv_rms + (size_t)b * Tn;
  const T* xb = x + ob;
  // g[t, c8 .. c8 + 7] = dxn + the conv's transpose
  auto gvec = [&](int t, int c8, const float (&tq)[KA][8], const float (&tk)[KA][8], const float (&tv)[KA][8],
                  float (&g)[8]) {
    ld8(dxn + ob + (size_t)t * dim + c8, g);
    if constexpr (KT > 0) {
#pragma unroll
      for (int j = 0; j < KT; ++j) {
        const int u = t - j + pad;   // xn[t] feeds output u
        if (u < 0 || u >= Tn) continue;
        float a[8], c[8], d[8];
        const size_t ou = ob + (size_t)u * dim + c8;
        ld8(dqi + ou, a);
        ld8(dki + ou, c);
        ld8(dvi + ou, d);
#pragma unroll
        for (int e = 0; e < 8; ++e) g[e] += tq[j][e] * a[e] + tk[j][e] * c[e] + tv[j][e] * d[e];
      }
    }
  };
  // sums sred[*][0 .. n) over the waves into dst (n = 8 * 64 * per-lane values of this 512-channel chunk)
  auto wave_reduce_store = [&](float* dst, int n) {
    __syncthreads();
    for (int i = tid; i < n; i += pro::kThreads) {
      float acc = 0.f;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) acc += sred[ww][i];
      dst[i] = acc;
    }
    __syncthreads();
  };
  float dot[TW];
#pragma unroll
  for (int i = 0; i < TW; ++i) dot[i] = 0.f;
  // pass A
  for (int cb = 0; cb < dim; cb += 512) {
    const int c8 = cb + lane * 8;
    const bool on = c8 < dim;
    float dw[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (on) {
      float wv8[8], tq[KA][8], tk[KA][8], tv[KA][8];
      ld8(wn + c8, wv8);
      if constexpr (KT > 0) {
        load_taps<T, KT>(wq, c8, tq);
        load_taps<T, KT>(wk, c8, tk);
        load_taps<T, KT>(wv, c8, tv);
      }
#pragma unroll
      for (int i = 0; i < TW; ++i) {
        const int t = t0 + i;
        if (t >= t1) break;
        float g[8], xv[8];
        gvec(t, c8, tq, tk, tv, g);
        ld8(xb + (size_t)t * dim + c8, xv);
        const float it = inv[t];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          dw[e] += g[e] * xv[e] * it;
          dot[i] += wv8[e] * g[e] * xv[e];
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) sred[w][lane * 8 + e] = dw[e];
    wave_reduce_store(dwn_part + prow * dim + cb, min(512, dim - cb));
  }
#pragma unroll
  for (int i = 0; i < TW; ++i) dot[i] = wave_sum(dot[i]);
  // pass B: dx
  for (int c8 = lane * 8; c8 < dim; c8 += 512) {
    float wv8[8], tq[KA][8], tk[KA][8], tv[KA][8];
    ld8(wn + c8, wv8);
    if constexpr (KT > 0) {
      load_taps<T, KT>(wq, c8, tq);
      load_taps<T, KT>(wk, c8, tk);
      load_taps<T, KT>(wv, c8, tv);
    }
#pragma unroll
    for (int i = 0; i < TW; ++i) {
      const int t = t0 + i;
      if (t >= t1) break;
      float g[8], xv[8];
      gvec(t, c8, tq, tk, tv, g);
      ld8(xb + (size_t)t * dim + c8, xv);
      const float it = inv[t], c3 = it * it * it * dot[i] / (float)dim;
#pragma unroll
      for (int e = 0; e < 8; ++e) g[e] = it * wv8[e] * g[e] - xv[e] * c3;
      st8(dx + ob + (size_t)t * dim + c8, g);
    }
  }
  // pass C: tap partials, output t reads xn[t + j - pad]; one conv at a time through LDS
  if constexpr (KT > 0) {
    for (int cb = 0; cb < dim; cb += 512) {
      const int c8 = cb + lane * 8;
      const bool on = c8 < dim;
      float wv8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (on) ld8(wn + c8, wv8);
#pragma unroll
      for (int which = 0; which < 3; ++which) {
        const T* dc = which == 0 ? dqi : (which == 1 ? dki : dvi);
        float gt[KT][8];
#pragma unroll
        for (int j = 0; j < KT; ++j)
#pragma unroll
          for (int e = 0; e < 8; ++e) gt[j][e] = 0.f;
        if (on) {
          for (int t = t0; t < t1; ++t) {
            float dd[8];
            ld8(dc + ob + (size_t)t * dim + c8, dd);
#pragma unroll
            for (int j = 0; j < KT; ++j) {
              const int s_ = t + j - pad;
              if (s_ < 0 || s_ >= Tn) continue;
              float xs[8];
              ld8(xb + (size_t)s_ * dim + c8, xs);
              const float is = inv[s_];
#pragma unroll
              for (int e = 0; e < 8; ++e) gt[j][e] += dd[e] * xs[e] * is * wv8[e];
            }
          }
        }
        // layout of a conv's partial: [dim][K] -> this chunk is 512 K contiguous values
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
          for (int j = 0; j < KT; ++j) sred[w][(lane * 8 + e) * KT + j] = gt[j][e];
        wave_reduce_store(dwc_part + (prow * 3 + which) * dim * KT + (size_t)cb * KT, min(512, dim - cb) * KT);
      }
    }
  }
}

// The same adjoint in one pass over the tokens, for dim <= 512 and conv_k <= 4 (the cell's shapes):
// a workgroup of two waves per 16-token block, lane l of wave w owning channels c = 4 (64 w + l) ..
// c + 3. The conv's transpose is scattered as each row u of dq_in / dk_in / dv_in arrives: it adds
// taps[j] * dconv[u] to g of token u + j - pad, so that g of token u - pad is complete after row u;
// that token is then finished at once (the RMSNorm adjoint's dot product summed over the lanes and
// the two waves, dx, the norm-weight partial), and row u also feeds the tap partials with the x rows
// u - pad .. u - pad + K - 1 held in a register window. Every input row is read once per block
// (plus the K - 1 halo rows), with the loads of step u + 2 in flight during step u; rows outside
// [0, T) read as zeros through the buffer range check (the convs' zero padding). Same partial layout
// as k_pro_bwd (one row per 16-token block).
namespace pw {
constexpr int kWaves = 2, kThreads = 64 * kWaves, kCh = 4;   // channels per lane
constexpr int kMaxDim = kThreads * kCh;                      // 512
}

// Four consecutive elements through a buffer resource, as fp32. The fp32 form converts the whole
// 16-byte vector at once: hipcc 7.2 narrows a raw buffer load whose vector elements are bit-cast to
// float one by one to a single dword (the other three elements then hold stale registers).
typedef float f32x4v __attribute__((ext_vector_type(4)));
template <typename T>
__device__ __forceinline__ float4 ld4_rs(rsrc_t r, uint32_t off) {
  if constexpr (sizeof(T) == 2) {
    const u32x2v u = bld8(r, off);
    return make_float4(__builtin_bit_cast(float, u[0] << 16), __builtin_bit_cast(float, u[0] & 0xffff0000u),
                       __builtin_bit_cast(float, u[1] << 16), __builtin_bit_cast(float, u[1] & 0xffff0000u));
  } else {
    const f32x4v v = __builtin_bit_cast(f32x4v, bld16(r, off));
    return make_float4(v[0], v[1], v[2], v[3]);
  }
}
template <typename T>
__device__ __forceinline__ void st4_rs(rsrc_t r, uint32_t off, const float (&v)[4]) {
  if constexpr (sizeof(T) == 2) {
    u32x2v u;
    u[0] = pack_bf16x2(v[0], v[1]);
    u[1] = pack_bf16x2(v[2], v[3]);
    bst8(r, off, u);
  } else {
    const f32x4v f = {v[0], v[1], v[2], v[3]};
    bst16(r, off, __builtin_bit_cast(u32x4v, f));
  }
}

template <typename T, int KT>
__global__ __launch_bounds__(pw::kThreads) void k_pro_bwd_win(int Tn, int dim, const T* __restrict__ x,
                                                              const T* __restrict__ wn, const T* __restrict__ wq,
                                                              const T* __restrict__ wk, const T* __restrict__ wv,
                                                              const float* __restrict__ inv_rms,
                                                              const T* __restrict__ dxn, const T* __restrict__ dqi,
                                                              const T* __restrict__ dki, const T* __restrict__ dvi,
                                                              T* __restrict__ dx, float* __restrict__ dwn_part,
                                                              float* __restrict__ dwc_part) {
  constexpr int pad = KT / 2, KA = KT > 0 ? KT : 1, E = (int)sizeof(T);
  __shared__ float sdot[2][pw::kWaves];   // per-wave partial dot products, by step parity
  const int lane = lane_id(), w = wave_id();
  const int b = blockIdx.y, blk = blockIdx.x, ntb = gridDim.x;
  const int t0 = blk * pro::kTok, t1 = min(Tn, t0 + pro::kTok);
  const int c = pw::kCh * (64 * w + lane);
  const bool on = c < dim;
  const size_t ob = (size_t)b * Tn * dim, prow = (size_t)b * ntb + blk;
  const uint32_t nbytes = (uint32_t)((size_t)Tn * dim * E);
  const float* inv = inv_rms + (size_t)b * Tn;
  const rsrc_t rx = make_rsrc(x + ob, nbytes), rdxn = make_rsrc(dxn + ob, nbytes), rdx = make_rsrc(dx + ob, nbytes);
  const rsrc_t rq = make_rsrc(KT ? dqi + ob : x, KT ? nbytes : 0u), rk = make_rsrc(KT ? dki + ob : x, KT ? nbytes : 0u),
               rv = make_rsrc(KT ? dvi + ob : x, KT ? nbytes : 0u);
  // byte offset of this lane's channels in row r (rows < 0 wrap past the range and read zeros)
  auto roff = [&](int r) { return on ? (uint32_t)((r * dim + c) * E) : kOob; };
  auto inv_at = [&](int r) { return (r >= 0 && r < Tn) ? inv[r] : 0.f; };

  float wn4[4] = {0.f, 0.f, 0.f, 0.f}, tap[3][KA][4];
  if (on) {
#pragma unroll
    for (int e = 0; e < 4; ++e) wn4[e] = to_f32(wn[c + e]);
  }
#pragma unroll
  for (int h = 0; h < 3; ++h)
#pragma unroll
    for (int j = 0; j < KA; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const T* tw = h == 0 ? wq : (h == 1 ? wk : wv);
        tap[h][j][e] = (KT > 0 && on) ? to_f32(tw[(size_t)(c + e) * KT + j]) : 0.f;
      }
  float gt[3][KA][4], dw4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int h = 0; h < 3; ++h)
#pragma unroll
    for (int j = 0; j < KA; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) gt[h][j][e] = 0.f;
  // windows: gw[m] = g of token u - pad + m (scatter targets), xw[m] / iw[m] = x row u - pad + m
  float gw[KA][4], xw[KA][4], iw[KA];
#pragma unroll
  for (int m = 0; m < KA; ++m) {
    iw[m] = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) gw[m][e] = xw[m][e] = 0.f;
  }
  // steps u in [ub, ue]: conv rows (KT > 0) or tokens (KT = 0)
  const int ub = KT ? t0 + pad - KT + 1 : t0, ue = KT ? t1 - 1 + pad : t1 - 1;
  if constexpr (KT > 0) {   // x rows ub - pad .. ub - pad + KT - 2 (the last window row comes with step ub)
#pragma unroll
    for (int m = 0; m + 1 < KT; ++m) {
      const float4 v = ld4_rs<T>(rx, roff(ub - pad + m));
      xw[m][0] = v.x; xw[m][1] = v.y; xw[m][2] = v.z; xw[m][3] = v.w;
      iw[m] = inv_at(ub - pad + m);
    }
  }
  // inputs of one step: conv rows u, x row u - pad + K - 1 (its inverse RMS), dxn of token u - pad
  struct Stage {
    float4 q, k, v, x, d;
    float i;
  };
  auto sload = [&](Stage& st, int u) {
    const int xr = u - pad + KA - 1, tk = u - pad;
    if constexpr (KT > 0) {
      st.q = ld4_rs<T>(rq, roff(u));
      st.k = ld4_rs<T>(rk, roff(u));
      st.v = ld4_rs<T>(rv, roff(u));
    }
    st.x = ld4_rs<T>(rx, roff(xr));
    st.i = inv_at(xr);
    st.d = ld4_rs<T>(rdxn, roff(tk));
  };
  auto step = [&](int u, Stage& st) {
    const int tk = u - pad;
    {   // newest window row
      xw[KA - 1][0] = st.x.x; xw[KA - 1][1] = st.x.y; xw[KA - 1][2] = st.x.z; xw[KA - 1][3] = st.x.w;
      iw[KA - 1] = st.i;
    }
    if constexpr (KT > 0) {
      const float dq[4] = {st.q.x, st.q.y, st.q.z, st.q.w}, dk[4] = {st.k.x, st.k.y, st.k.z, st.k.w},
                  dv[4] = {st.v.x, st.v.y, st.v.z, st.v.w};
#pragma unroll
      for (int j = 0; j < KT; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) gw[j][e] += tap[0][j][e] * dq[e] + tap[1][j][e] * dk[e] + tap[2][j][e] * dv[e];
      if (u >= t0 && u < t1) {   // tap partials of output row u: xn rows u - pad + j
#pragma unroll
        for (int j = 0; j < KT; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float xn = xw[j][e] * iw[j] * wn4[e];
            gt[0][j][e] += dq[e] * xn;
            gt[1][j][e] += dk[e] * xn;
            gt[2][j][e] += dv[e] * xn;
          }
      }
    }
    if (tk >= t0 && tk < t1) {   // token tk is complete: finish it (uniform over the workgroup)
      const float dd[4] = {st.d.x, st.d.y, st.d.z, st.d.w};
      float g[4], pd = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        g[e] = gw[0][e] + dd[e];
        pd += wn4[e] * g[e] * xw[0][e];
      }
      pd = wave_sum(pd);
      const int par = tk & 1;
      if (lane == 0) sdot[par][w] = pd;
      __syncthreads();
      float dot = 0.f;
#pragma unroll
      for (int ww = 0; ww < pw::kWaves; ++ww) dot += sdot[par][ww];
      const float it = iw[0], c3 = it * it * it * dot / (float)dim;
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        dw4[e] += g[e] * xw[0][e] * it;
        o[e] = it * wn4[e] * g[e] - xw[0][e] * c3;
      }
      if (on) st4_rs<T>(rdx, roff(tk), o);
    }
    // shift the windows by one token
#pragma unroll
    for (int m = 0; m + 1 < KA; ++m) {
      iw[m] = iw[m + 1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        gw[m][e] = gw[m + 1][e];
        xw[m][e] = xw[m + 1][e];
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) gw[KA - 1][e] = 0.f;
    sload(st, u + 2);   // past ue: rows of the next block or past T (zeros), never used
  };
  Stage sa, sb;
  sload(sa, ub);
  sload(sb, ub + 1);
  for (int u = ub; u <= ue; u += 2) {
    step(u, sa);
    if (u + 1 <= ue) step(u + 1, sb);
  }
  if (on) {
    *reinterpret_cast<float4*>(dwn_part + prow * dim + c) = make_float4(dw4[0], dw4[1], dw4[2], dw4[3]);
    if constexpr (KT > 0) {   // [3][dim][K]: this lane's 4 K consecutive values per conv
#pragma unroll
      for (int h = 0; h < 3; ++h) {
        float* dst = dwc_part + ((prow * 3 + h) * dim + c) * KT;
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int j = 0; j < KT; ++j) dst[e * KT + j] = gt[h][j][e];
      }
    }
  }
}

// Sums of per-workgroup partials over their rows (the parameter gradients of the prologue and head
// kernels), several arrays in one launch: problem z is parts[z] [rows][cols[z]] fp32 -> outs[z]
// [cols[z]] in bf16 or fp32. Workgroup: 16 columns x 16 row groups; thread (group q, column c) sums
// rows q, q + 16, ... with four accumulators in a fixed pattern, and the sixteen group sums are
// added in order through LDS, so the result does not depend on scheduling (deterministic).
namespace ps {
constexpr int kMax = 8, kCols = 16, kGroups = 16;
struct List {
  const float* part[kMax];
  void* out[kMax];
  int cols[kMax];
  int off[kMax + 1];   // first flat column of each problem
  int bf16[kMax];
  int count;
};
}
__global__ __launch_bounds__(256) void k_partials_sum(int rows, ps::List L) {
  __shared__ float red[ps::kGroups][ps::kCols + 1];
  const int cl = threadIdx.x & (ps::kCols - 1), q = threadIdx.x / ps::kCols;
  const int fc = blockIdx.x * ps::kCols + cl;   // flat column
  int z = 0;
  while (z + 1 < L.count && fc >= L.off[z + 1]) ++z;
  const bool live = fc < L.off[L.count];
  const int c = fc - L.off[z];
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  if (live) {
    const float* p = L.part[z] + c;
    const size_t st = (size_t)L.cols[z];
    int r = q;
    for (; r + 3 * ps::kGroups < rows; r += 4 * ps::kGroups) {
      a0 += p[(size_t)r * st];
      a1 += p[(size_t)(r + ps::kGroups) * st];
      a2 += p[(size_t)(r + 2 * ps::kGroups) * st];
      a3 += p[(size_t)(r + 3 * ps::kGroups) * st];
    }
    for (; r < rows; r += ps::kGroups) a0 += p[(size_t)r * st];
  }
  red[q][cl] = (a0 + a1) + (a2 + a3);
  __syncthreads();
  if (q == 0 && live) {
    float sum = 0.f;
#pragma unroll
    for (int g = 0; g < ps::kGroups; ++g) sum += red[g][cl];
    if (L.bf16[z]) static_cast<bf16*>(L.out[z])[c] = static_cast<bf16>(sum);
    else static_cast<float*>(L.out[z])[c] = sum;
  }
}

// Threads per head row: d / 8 rounded up to a power of two (the extra threads hold zeros), so that
// a row's sums are xor shuffles within an aligned lane group.
__host__ __device__ __forceinline__ int heads_row_threads(int d) {
  int rl = 1;
  while (rl * 8 < d) rl <<= 1;
  return rl;
}
template <typename T>
__device__ __forceinline__ float row_sum8(float v, int rl) {   // sum over the rl threads of a row
  for (int m = rl >> 1; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

template <typename T>
__global__ __launch_bounds__(256) void k_heads_fwd(int Tn, int H, int d, int nG, const T* __restrict__ ql,
                                                   const T* __restrict__ kl, const T* __restrict__ vl,
                                                   const T* __restrict__ zl, const T* __restrict__ qg,
                                                   const T* __restrict__ kg, const T* __restrict__ bias,
                                                   T* __restrict__ q, T* __restrict__ k, T* __restrict__ v,
                                                   T* __restrict__ gates) {
  const int tb = blockIdx.x, bh = blockIdx.y, H_ = H, b = bh / H_, h = bh % H_, tid = threadIdx.x;
  const int rl = heads_row_threads(d), r = tid / rl, c8 = (tid % rl) * 8;
  const int t = tb * pro::kTok + r;
  const bool valid = t < Tn && c8 < d;
  const int HD = H * d, BH = gridDim.y;
  const float rs = rsqrtf((float)d);
  const size_t src = ((size_t)b * Tn + t) * HD + (size_t)h * d + c8;
  const size_t dst = ((size_t)bh * Tn + t) * d + c8;
#pragma unroll
  for (int which = 0; which < 3; ++which) {
    const T* in = which == 0 ? ql : (which == 1 ? kl : vl);
    T* out = which == 0 ? q : (which == 1 ? k : v);
    const T* gam = which == 0 ? qg : (which == 1 ? kg : nullptr);
    float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (valid) ld8(in + src, x);
    if (gam) {   // uniform
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
      ss = row_sum8<T>(ss, rl);
      const float scale = 1.f / fmaxf(sqrtf(ss) * rs, 1e-8f);
      float g[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (c8 < d) ld8(gam + (size_t)h * d + c8, g);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] *= scale * g[e];
    }
    if (valid) st8(out + dst, x);
  }
  // gates of this head: item i < nG * 16 -> gate i / 16, token i % 16
  for (int i = tid; i < nG * pro::kTok; i += blockDim.x) {
    const int g = i / pro::kTok, tt = tb * pro::kTok + i % pro::kTok;
    if (tt < Tn) {
      const float z = to_f32(zl[((size_t)b * Tn + tt) * nG * H + g * H + h]) + to_f32(bias[g * H + h]);
      gates[((size_t)g * BH + bh) * Tn + tt] = from_f32<T>(1.f / (1.f + __expf(-z)));
    }
  }
}

// Adjoint of k_heads_fwd: dq, dk, dv [(b h), T, d], dgates [nG][(b h), T] (null: zero) and the forward's
// gates -> dql, dkl, dvl [B, T, H d], dzl [B, T, nG H]; partials dqg_part, dkg_part [nwg][H][d] (when
// the norms exist) and dbias_part [nwg][nG H], nwg = B * ceil(T / 16): workgroup (token block tb,
// (b, h)) writes row b * ceil(T / 16) + tb, columns of head h.
//   y = x s gamma, s = 1 / max(r, 1e-8), r = |x| / sqrt(d):  dx = s gamma dy - x s^3 (x . gamma dy) / d  (r > 1e-8)
template <typename T>
__global__ __launch_bounds__(256) void k_heads_bwd(int Tn, int H, int d, int nG, const T* __restrict__ ql,
                                                   const T* __restrict__ kl, const T* __restrict__ qg,
                                                   const T* __restrict__ kg, const T* __restrict__ gates,
                                                   const T* __restrict__ dq, const T* __restrict__ dk,
                                                   const T* __restrict__ dv, const T* __restrict__ dgates,
                                                   T* __restrict__ dql, T* __restrict__ dkl, T* __restrict__ dvl,
                                                   T* __restrict__ dzl, float* __restrict__ dqg_part,
                                                   float* __restrict__ dkg_part, float* __restrict__ dbias_part) {
  __shared__ float sgp[2][pro::kTok][128 + 1];   // gamma-gradient terms per token row, q and k
  __shared__ float sbp[8][pro::kTok];            // bias-gradient terms per gate and token
  const int tb = blockIdx.x, bh = blockIdx.y, b = bh / H, h = bh % H, tid = threadIdx.x;
  const int rl = heads_row_threads(d), r = tid / rl, c8 = (tid % rl) * 8;
  const int t = tb * pro::kTok + r;
  const bool valid = t < Tn && c8 < d;
  const int HD = H * d, BH = gridDim.y, ntb = gridDim.x;
  const float rs = rsqrtf((float)d);
  const bool norm = qg != nullptr;
  const size_t xo = ((size_t)b * Tn + t) * HD + (size_t)h * d + c8;
  const size_t yo = ((size_t)bh * Tn + t) * d + c8;
#pragma unroll
  for (int which = 0; which < 3; ++which) {
    const T* dy = which == 0 ? dq : (which == 1 ? dk : dv);
    T* dxo = which == 0 ? dql : (which == 1 ? dkl : dvl);
    float gv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (valid) ld8(dy + yo, gv);
    if (which == 2 || !norm) {
      if (valid) st8(dxo + xo, gv);
      continue;
    }
    const T* in = which == 0 ? ql : kl;
    const T* gam = which == 0 ? qg : kg;
    float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, gm[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (valid) ld8(in + xo, x);
    if (c8 < d) ld8(gam + (size_t)h * d + c8, gm);
    float ss = 0.f, xu = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      ss += x[e] * x[e];
      xu += x[e] * gm[e] * gv[e];
    }
    ss = row_sum8<T>(ss, rl);
    xu = row_sum8<T>(xu, rl);
    const float r_ = sqrtf(ss) * rs;
    const float sc = 1.f / fmaxf(r_, 1e-8f);
    const float c3 = r_ > 1e-8f ? sc * sc * sc * xu / (float)d : 0.f;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o[e] = sc * gm[e] * gv[e] - x[e] * c3;
      if (c8 < d) sgp[which][r][c8 + e] = gv[e] * x[e] * sc;   // 0 for rows past T (x = 0)
    }
    if (valid) st8(dxo + xo, o);
  }
  // gates: dz = dg s (1 - s)
  for (int i = tid; i < nG * pro::kTok; i += blockDim.x) {
    const int g = i / pro::kTok, rr = i % pro::kTok, tt = tb * pro::kTok + rr;
    float dz = 0.f;
    if (tt < Tn) {
      const size_t go = ((size_t)g * BH + bh) * Tn + tt;
      const float sg = to_f32(gates[go]);
      const float dg = dgates ? to_f32(dgates[go]) : 0.f;
      dz = dg * sg * (1.f - sg);
      dzl[((size_t)b * Tn + tt) * nG * H + g * H + h] = from_f32<T>(dz);
    }
    sbp[g][rr] = dz;
  }
  __syncthreads();
  const size_t prow = (size_t)b * ntb + tb;
  if (norm) {
    for (int i = tid; i < 2 * d; i += blockDim.x) {
      const int which = i / d, c = i % d;
      float acc = 0.f;
#pragma unroll
      for (int rr = 0; rr < pro::kTok; ++rr) acc += sgp[which][rr][c];
      (which ? dkg_part : dqg_part)[prow * HD + (size_t)h * d + c] = acc;
    }
  }
  for (int g = tid; g < nG; g += blockDim.x) {
    float acc = 0.f;
#pragma unroll
    for (int rr = 0; rr < pro::kTok; ++rr) acc += sbp[g][rr];
    dbias_part[prow * nG * H + g * H + h] = acc;
  }
}

}  // namespace atlas

using namespace atlas;

namespace {
bool pro_shapes_ok(int B, int Tn, int dim, int K) {
  return B >= 1 && B <= 65535 && Tn >= 1 && dim >= 8 && dim <= (1 << 16) && dim % 8 == 0 && K >= 0 &&
         K <= pro::kMaxK;
}
bool heads_shapes_ok(int B, int Tn, int H, int d, int nG) {
  return B >= 1 && Tn >= 1 && H >= 1 && (int64_t)B * H <= 65535 && d >= 8 && d <= 128 && d % 8 == 0 && nG >= 0 &&
         nG <= 8;
}
}  // namespace

extern "C" {

int atlas_partials_sum(int count, int rows, const int* cols, const float* const* parts, void* const* outs,
                       const int* out_dtypes, void* stream) {
  using namespace atlas;
  if (count < 1 || count > ps::kMax || rows < 0) return ATLAS_MEM_ERR_SHAPE;
  if (!cols || !parts || !outs || !out_dtypes) return ATLAS_MEM_ERR_NULL;
  ps::List L = {};
  L.count = count;
  int64_t total = 0;
  for (int z = 0; z < count; ++z) {
    if (cols[z] < 1) return ATLAS_MEM_ERR_SHAPE;
    if (out_dtypes[z] != ATLAS_DT_BF16 && out_dtypes[z] != ATLAS_DT_F32) return ATLAS_MEM_ERR_DTYPE;
    if (!outs[z] || (rows > 0 && !parts[z])) return ATLAS_MEM_ERR_NULL;
    L.part[z] = parts[z];
    L.out[z] = outs[z];
    L.cols[z] = cols[z];
    L.bf16[z] = out_dtypes[z] == ATLAS_DT_BF16;
    L.off[z] = (int)total;
    total += cols[z];
    if (total >= ((int64_t)1 << 30)) return ATLAS_MEM_ERR_SHAPE;
  }
  L.off[count] = (int)total;
  const unsigned grid = (unsigned)((total + ps::kCols - 1) / ps::kCols);
  hipLaunchKernelGGL(k_partials_sum, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream), rows, L);
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

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
  for (const void* p : {x, norm_w, (const void*)xn, (const void*)q_in, (const void*)k_in, (const void*)v_in})
    if (reinterpret_cast<uintptr_t>(p) & 15) return ATLAS_MEM_ERR_ALIGN;
  const dim3 grid((seq_len + pro::kTok - 1) / pro::kTok, batch), block(pro::kThreads);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int K = conv ? conv_k : 0;
  auto go = [&](auto tag, auto kt) {
    using T = decltype(tag);
    constexpr int KT = decltype(kt)::value;
    hipLaunchKernelGGL((k_pro_fwd<T, KT>), grid, block, 0, s, seq_len, dim, eps, (const T*)x, (const T*)norm_w,
                       (const T*)wq, (const T*)wk, (const T*)wv, (T*)xn, (T*)q_in, (T*)k_in, (T*)v_in, inv_rms);
  };
  auto by_k = [&](auto tag) {
    switch (K) {
      case 0: go(tag, std::integral_constant<int, 0>{}); break;
      case 2: go(tag, std::integral_constant<int, 2>{}); break;
      case 3: go(tag, std::integral_constant<int, 3>{}); break;
      case 4: go(tag, std::integral_constant<int, 4>{}); break;
      case 5: go(tag, std::integral_constant<int, 5>{}); break;
      case 6: go(tag, std::integral_constant<int, 6>{}); break;
      case 7: go(tag, std::integral_constant<int, 7>{}); break;
      default: go(tag, std::integral_constant<int, 8>{}); break;
    }
  };
  if (dtype == ATLAS_DT_BF16) by_k(bf16{});
  else by_k(float{});
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
  for (const void* p : {x, norm_w, dxn, dq_in, dk_in, dv_in, (const void*)dx})
    if (reinterpret_cast<uintptr_t>(p) & 15) return ATLAS_MEM_ERR_ALIGN;
  const dim3 grid((seq_len + pro::kTok - 1) / pro::kTok, batch), block(pro::kThreads);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int K = conv ? conv_k : 0;
  const size_t esize = dtype == ATLAS_DT_BF16 ? 2 : 4;
  // one pass over the tokens where the per-lane windows fit (dim <= 512, conv_k <= 4)
  const bool win = dim <= pw::kMaxDim && K <= 4 && (size_t)seq_len * dim * esize < ((size_t)1 << 31);
  auto go = [&](auto tag, auto kt) {
    using T = decltype(tag);
    constexpr int KT = decltype(kt)::value;
    if constexpr (KT <= 4) {
      if (win) {
        hipLaunchKernelGGL((k_pro_bwd_win<T, KT>), grid, dim3(pw::kThreads), 0, s, seq_len, dim, (const T*)x,
                           (const T*)norm_w, (const T*)wq, (const T*)wk, (const T*)wv, inv_rms, (const T*)dxn,
                           (const T*)dq_in, (const T*)dk_in, (const T*)dv_in, (T*)dx, dnorm_w_part, dconv_part);
        return;
      }
    }
    hipLaunchKernelGGL((k_pro_bwd<T, KT>), grid, block, 0, s, seq_len, dim, (const T*)x, (const T*)norm_w,
                       (const T*)wq, (const T*)wk, (const T*)wv, inv_rms, (const T*)dxn, (const T*)dq_in,
                       (const T*)dk_in, (const T*)dv_in, (T*)dx, dnorm_w_part, dconv_part);
  };
  auto by_k = [&](auto tag) {
    switch (K) {
      case 0: go(tag, std::integral_constant<int, 0>{}); break;
      case 2: go(tag, std::integral_constant<int, 2>{}); break;
      case 3: go(tag, std::integral_constant<int, 3>{}); break;
      case 4: go(tag, std::integral_constant<int, 4>{}); break;
      case 5: go(tag, std::integral_constant<int, 5>{}); break;
      case 6: go(tag, std::integral_constant<int, 6>{}); break;
      case 7: go(tag, std::integral_constant<int, 7>{}); break;
      default: go(tag, std::integral_constant<int, 8>{}); break;
    }
  };
  if (dtype == ATLAS_DT_BF16) by_k(bf16{});
  else by_k(float{});
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
  for (const void* p : {ql, kl, vl, q_gamma, k_gamma, (const void*)q, (const void*)k, (const void*)v})
    if (reinterpret_cast<uintptr_t>(p) & 15) return ATLAS_MEM_ERR_ALIGN;
  const dim3 grid((seq_len + pro::kTok - 1) / pro::kTok, batch * heads), block(pro::kTok * heads_row_threads(d));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == ATLAS_DT_BF16)
    hipLaunchKernelGGL(k_heads_fwd<bf16>, grid, block, 0, s, seq_len, heads, d, n_gates, (const bf16*)ql,
                       (const bf16*)kl, (const bf16*)vl, (const bf16*)zl, (const bf16*)q_gamma, (const bf16*)k_gamma,
                       (const bf16*)gate_bias, (bf16*)q, (bf16*)k, (bf16*)v, (bf16*)gates);
  else
    hipLaunchKernelGGL(k_heads_fwd<float>, grid, block, 0, s, seq_len, heads, d, n_gates,
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
  for (const void* p : {ql, kl, q_gamma, k_gamma, dq, dk, dv, (const void*)dql, (const void*)dkl, (const void*)dvl})
    if (reinterpret_cast<uintptr_t>(p) & 15) return ATLAS_MEM_ERR_ALIGN;
  const dim3 grid((seq_len + pro::kTok - 1) / pro::kTok, batch * heads), block(pro::kTok * heads_row_threads(d));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == ATLAS_DT_BF16)
    hipLaunchKernelGGL(k_heads_bwd<bf16>, grid, block, 0, s, seq_len, heads, d, n_gates,
                       (const bf16*)ql, (const bf16*)kl, (const bf16*)q_gamma, (const bf16*)k_gamma,
                       (const bf16*)gates, (const bf16*)dq, (const bf16*)dk, (const bf16*)dv, (const bf16*)dgates,
                       (bf16*)dql, (bf16*)dkl, (bf16*)dvl, (bf16*)dzl, dq_gamma_part, dk_gamma_part, dbias_part);
  else
    hipLaunchKernelGGL(k_heads_bwd<float>, grid, block, 0, s, seq_len, heads, d, n_gates,
                       (const float*)ql, (const float*)kl, (const float*)q_gamma, (const float*)k_gamma,
                       (const float*)gates, (const float*)dq, (const float*)dk, (const float*)dv, (const float*)dgates,
                       (float*)dql, (float*)dkl, (float*)dvl, (float*)dzl, dq_gamma_part, dk_gamma_part, dbias_part);
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

}  // extern "C"
