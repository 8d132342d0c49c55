// bufwalk.hip - a carried Omega buffer on the specialised bf16, d = 64 walks.
//
// The buffer's slots B_s [e-1][D][D] (slot 0 the oldest) stand for the e - 1 sources before token 0:
// where a token's source term is delta_s phi_s^T, a buffer source's is B_s (rnn_memory.py:673-687,
// the window over [__omega_buf; gated]). Source slot s of the first chunk is token s - (e - 1), so
// the buffer sources are the halo slots s < e - 1 of chunk 0, whose token rows the walks read as
// zeros. Every buffer term is linear in B and lies in chunk 0 (the later chunks see it through the
// state), so the walks keep their chunk code and take these terms from two small launches:
//
//   k_buf_fwd (before the walks), with the forward chunk's coefficient record and Ws block:
//     y corrections     yc[t] = -sum_s Ws[s, t-1] B_s psi_t                      (t < 64)
//     state corrections dS_end = -sum_s Ws[s, end] B_s,  dZ_end = sum_s Wz[s, end] B_s, and the same
//                       after token Lmid - 1 (the saved backward-chunk boundary); Z terms only with
//                       momentum. k_walk_full adds them at the end of chunk 0 and to the y of chunk
//                       0's targets; carried through segment 0's later chunks (their end scalars a,
//                       kappa, b), the end terms are added to segment 0's aggregate by the segment scan.
//   k_buf_bwd (after k_walk_bwd, before the scalar chain), with the backward chunk's records and the
//   chunk-0 end adjoint (dS_e, dZ_e) the reverse walk leaves in buf_adj:
//     d buffer_in[s] = Wz[s, end] dZ_e - Ws[s, end] dS_e - sum_q Ws[s, q-1] dy_q psi_q^T
//     records of chunk 0: hS[s] += <dS_e, B_s>, hZ[s] += <dZ_e, B_s>, Lm[q][s] += dy_q^T B_s psi_q
//     dq[q] += -(sum_s Ws[s, q-1] B_s^T dy_q) * map'(q)                             (q < 32)
//   (the same terms as the general kernels' first-chunk buffer code, seg_fwd.h / seg_bwd.hip).
// Workgroups of 256 threads; fp32 arithmetic on the fp32 buffer.
#include "mem_common.h"
#include "mem_params.h"
#include "seg_common.h"

#include <algorithm>

namespace atlas {

namespace {

constexpr int kBwThreads = 256;
constexpr int D = bufw::D;

template <int CH>
struct RecOff {
  static constexpr int SPM = CoefRec<CH>::SPM;
  static constexpr int ACOEF = 0, KCOEF = CH, ENDC = 2 * CH, WSEND = 2 * CH + 4, WZEND = WSEND + SPM,
                       WSMID = WZEND + SPM, WZMID = WSMID + SPM;
};

__device__ __forceinline__ float bf16f(bf16 x) { return static_cast<float>(x); }

// one buffer slot [D][D] fp32 -> LDS (pitch D + 1)
__device__ __forceinline__ void stage_slot(float (*sB)[D + 1], const float* Bs) {
  for (int v = threadIdx.x; v < D * D / 4; v += kBwThreads) {
    const float4 x = reinterpret_cast<const float4*>(Bs)[v];
    const int i = (4 * v) / D, k = (4 * v) % D;
    sB[i][k] = x.x; sB[i][k + 1] = x.y; sB[i][k + 2] = x.z; sB[i][k + 3] = x.w;
  }
}

// grid (CHF / 16, BH): workgroup x forms the y corrections of tokens 16 x .. 16 x + 15 and a quarter
// of the state corrections (elements 1024 x ..). G0: the chunks of segment 0 when there are several
// segments (the end terms are carried through its chunks 1 .. G0 - 1 for its aggregate), else 0.
__global__ __launch_bounds__(kBwThreads) void k_buf_fwd(const Geom g, const FwdPtrs<bf16> a, const float* __restrict__ coef,
                                                        const bf16* __restrict__ wsh, float* __restrict__ corr, int G0) {
  if (geom_skip(g)) return;
  constexpr int CH = bufw::CHF, TG = 16;
  using R = RecOff<CH>;
  __shared__ float sB[D][D + 1];
  __shared__ float sp[TG][D + 1];
  const int tid = threadIdx.x, bh = blockIdx.y, xg = blockIdx.x;
  const int H = g.H, L = min(g.T, CH);
  const float* rec = coef + (size_t)bh * g.nc * CoefRec<CH>::SIZE;       // chunk 0
  const bf16* w0 = wsh + (size_t)bh * g.nc * CH * R::SPM;                 // chunk 0: Ws rows [t][s]
  float* out = corr + (size_t)bh * bufw::kCorrFloats;
  for (int idx = tid; idx < TG * D; idx += kBwThreads) {
    const int t = TG * xg + idx / D, k = idx % D;
    sp[idx / D][k] = t < L ? ld_map(a.q, ((size_t)bh * g.T + t) * D + k, g.map_mode, g.map_deg) : 0.f;
  }
  const int tt = tid >> 4, il = tid & 15, t = TG * xg + tt;   // y rows il + 16 r of token t
  const int eb = xg * (D * D / 4) + 4 * tid;                   // state elements eb .. eb + 3
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  float se[4] = {0.f, 0.f, 0.f, 0.f}, ze[4] = {0.f, 0.f, 0.f, 0.f};
  float sm[4] = {0.f, 0.f, 0.f, 0.f}, zm[4] = {0.f, 0.f, 0.f, 0.f};
  const float* Bb = a.buf_in + (size_t)bh * H * D * D;
  for (int s = 0; s < H; ++s) {
    const float* Bs = Bb + (size_t)s * D * D;
    __syncthreads();   // the previous slot's readers are done
    stage_slot(sB, Bs);
    __syncthreads();
    const float w = t < L ? bf16f(w0[(size_t)t * R::SPM + s]) : 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = il + 16 * r;
      float dot = 0.f;
#pragma unroll 16
      for (int k = 0; k < D; ++k) dot += sB[i][k] * sp[tt][k];
      acc[r] -= w * dot;
    }
    const float4 b = *reinterpret_cast<const float4*>(Bs + eb);
    const float bv[4] = {b.x, b.y, b.z, b.w};
    const float ws = rec[R::WSEND + s], wz = rec[R::WZEND + s], wsm = rec[R::WSMID + s], wzm = rec[R::WZMID + s];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      se[r] -= ws * bv[r];
      ze[r] += wz * bv[r];
      sm[r] -= wsm * bv[r];
      zm[r] += wzm * bv[r];
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) out[bufw::Y + t * D + il + 16 * r] = acc[r];   // zero past L
  const float zk = g.momentum ? 1.f : 0.f;
  // through chunks 1 .. G0 - 1 with no input: dS <- a dS - kappa dZ, dZ <- b dZ, i.e. at segment 0's
  // end dS_A = pa dS - pk dZ, dZ_A = pb dZ
  float pa = 1.f, pk = 0.f, pb = zk;
  for (int c = 1; c < G0; ++c) {
    const float* rc = rec + (size_t)c * CoefRec<CH>::SIZE;
    const float ca = rc[R::ENDC], ck = rc[R::ENDC + 1], cb = rc[R::ENDC + 2];
    pk = ca * pk + ck * pb;
    pa = ca * pa;
    pb = zk * cb * pb;
  }
  *reinterpret_cast<float4*>(out + bufw::SE + eb) = make_float4(se[0], se[1], se[2], se[3]);
  *reinterpret_cast<float4*>(out + bufw::ZE + eb) = make_float4(zk * ze[0], zk * ze[1], zk * ze[2], zk * ze[3]);
  *reinterpret_cast<float4*>(out + bufw::SM + eb) = make_float4(sm[0], sm[1], sm[2], sm[3]);
  *reinterpret_cast<float4*>(out + bufw::ZM + eb) = make_float4(zk * zm[0], zk * zm[1], zk * zm[2], zk * zm[3]);
  float au[4], av[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    au[r] = pa * se[r] - pk * zk * ze[r];
    av[r] = pb * ze[r];
  }
  *reinterpret_cast<float4*>(out + bufw::AU + eb) = make_float4(au[0], au[1], au[2], au[3]);
  *reinterpret_cast<float4*>(out + bufw::AV + eb) = make_float4(av[0], av[1], av[2], av[3]);
}

// grid (e, BH): workgroup s < e - 1 forms d buffer_in[s] and slot s's record terms; workgroup e - 1
// the dq terms of the first backward chunk (every slot).
__global__ __launch_bounds__(kBwThreads) void k_buf_bwd(const Geom g, const BwdPtrs<bf16> a, const BwdSegPtrs p) {
  if (geom_skip(g)) return;
  constexpr int CH = bufw::CHB;
  using R = RecOff<CH>;
  using SB = ScalarBlock<CH>;
  __shared__ float sB[D][D + 1];
  __shared__ float sdy[CH][D + 1];
  __shared__ float sps[CH][D + 1];
  __shared__ float sw[CH];
  __shared__ float sred[2][kBwThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, bh = blockIdx.y, s = blockIdx.x;
  const int H = g.H, Lq = min(g.T, CH);
  const size_t tb = (size_t)bh * g.T;
  const float* rec = p.coef + (size_t)bh * g.nc * CoefRec<CH>::SIZE;                       // chunk 0
  const bf16* w0 = reinterpret_cast<const bf16*>(p.wsh) + (size_t)bh * g.nc * CH * R::SPM;  // chunk 0
  float* blk = p.scal + (size_t)bh * g.nc * SB::SIZE;                                       // chunk 0
  const float* Bb = a.buf_in + (size_t)bh * H * D * D;
  for (int idx = tid; idx < CH * D; idx += kBwThreads) {
    const int q = idx / D, k = idx % D;
    sdy[q][k] = q < Lq ? bf16f(a.dy[(tb + q) * D + k]) : 0.f;
    if (s < H) sps[q][k] = q < Lq ? ld_map(a.q, (tb + q) * D + k, g.map_mode, g.map_deg) : 0.f;
  }
  if (s == H) {   // dq[q][k] += -(sum_s w(q, s) sum_i B_s[i][k] dy_q[i]) map'(q[q][k]); lane: q, columns k
    const int q = tid >> 3, kl = tid & 7;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int sl = 0; sl < H; ++sl) {
      __syncthreads();
      stage_slot(sB, Bb + (size_t)sl * D * D);
      __syncthreads();
      const float w = q < Lq ? bf16f(w0[(size_t)q * R::SPM + sl]) : 0.f;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int k = kl + 8 * r;
        float dot = 0.f;
#pragma unroll 16
        for (int i = 0; i < D; ++i) dot += sB[i][k] * sdy[q][i];
        acc[r] -= w * dot;
      }
    }
    if (q < Lq) {
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int k = kl + 8 * r;
        const size_t o = (tb + q) * D + k;
        const float mg = g.map_mode == MAP_ELEMENTWISE ? poly_map_grad(bf16f(a.q[o]), g.map_deg) : 1.f;
        a.dq[o] = from_f32<bf16>(bf16f(a.dq[o]) + acc[r] * mg);
      }
    }
    return;   // workgroup-uniform
  }
  // slot s: B_s, the weights w(q, s)
  stage_slot(sB, Bb + (size_t)s * D * D);
  if (tid < CH) sw[tid] = tid < Lq ? bf16f(w0[(size_t)tid * R::SPM + s]) : 0.f;
  __syncthreads();
  // d buffer_in[s] and <dS_e, B_s>, <dZ_e, B_s>; thread: row i, columns kb .. kb + 15
  {
    const int i = tid >> 2, kb = (tid & 3) * 16;
    const float* dSe = p.buf_adj + (size_t)bh * bufw::kAdjFloats;
    const float* dZe = dSe + D * D;
    const float ws = rec[R::WSEND + s], wz = rec[R::WZEND + s];
    float acc[16];
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) acc[kk] = 0.f;
    for (int q = 0; q < CH; ++q) {
      const float x = sw[q] * sdy[q][i];
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) acc[kk] += x * sps[q][kb + kk];
    }
    float hs = 0.f, hz = 0.f;
    float* dst = a.dbuf_in + (((size_t)bh * H + s) * D + i) * D + kb;
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      const float4 es = *reinterpret_cast<const float4*>(dSe + i * D + kb + 4 * k4);
      const float4 ez = *reinterpret_cast<const float4*>(dZe + i * D + kb + 4 * k4);
      const float vs[4] = {es.x, es.y, es.z, es.w}, vz[4] = {ez.x, ez.y, ez.z, ez.w};
      float o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float b = sB[i][kb + 4 * k4 + r];
        hs += vs[r] * b;
        hz += vz[r] * b;
        o[r] = wz * vz[r] - ws * vs[r] - acc[4 * k4 + r];
      }
      *reinterpret_cast<float4*>(dst + 4 * k4) = make_float4(o[0], o[1], o[2], o[3]);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      hs += __shfl_xor(hs, off, 64);
      hz += __shfl_xor(hz, off, 64);
    }
    if (lane == 0) { sred[0][wv] = hs; sred[1][wv] = hz; }
  }
  // Lm[q][s] += dy_q^T B_s psi_q; thread: token q, rows il + 8 r
  {
    const int q = tid >> 3, il = tid & 7;
    float v = 0.f;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int i = il + 8 * r;
      float dot = 0.f;
#pragma unroll 16
      for (int k = 0; k < D; ++k) dot += sB[i][k] * sps[q][k];
      v += sdy[q][i] * dot;
    }
    v += __shfl_xor(v, 1, 64);
    v += __shfl_xor(v, 2, 64);
    v += __shfl_xor(v, 4, 64);
    if (il == 0 && q < Lq) blk[SB::LM + q * SB::SPM + s] += v;
  }
  __syncthreads();
  if (tid == 0) {
    float hs = 0.f, hz = 0.f;
#pragma unroll
    for (int w = 0; w < kBwThreads / 64; ++w) { hs += sred[0][w]; hz += sred[1][w]; }
    blk[SB::HS + s] += hs;
    blk[SB::HZ + s] += hz;
  }
}

}  // namespace

hipError_t launch_buf_fwd(const Geom& g, const FwdPtrs<bf16>& a, const SegGeom& sg, const float* coef, const bf16* wsh,
                          float* corr, hipStream_t stream) {
  const int G0 = sg.nseg > 1 ? std::min(sg.G, g.nc) : 0;
  hipLaunchKernelGGL(k_buf_fwd, dim3(bufw::CHF / 16, g.BH), dim3(kBwThreads), 0, stream, g, a, coef, wsh, corr, G0);
  return hipGetLastError();
}

hipError_t launch_buf_bwd(const Geom& g, const BwdPtrs<bf16>& a, const BwdSegPtrs& p, hipStream_t stream) {
  hipLaunchKernelGGL(k_buf_bwd, dim3(g.e, g.BH), dim3(kBwThreads), 0, stream, g, a, p);
  return hipGetLastError();
}

}  // namespace atlas
