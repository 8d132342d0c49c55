// bufwalk.hip - a carried Omega buffer on the specialised bf16, d = 64 walks.
//
// The buffer's slots B_s [e-1][D][D] (slot 0 the oldest) stand for the e - 1 sources before token 0:
// where a token's source term is delta_s phi_s^T, a buffer source's is B_s (rnn_memory.py:673-687,
// the window over [__omega_buf; gated]). Source slot s of the first chunk is token s - (e - 1), so
// the buffer sources are the halo slots s < e - 1 of chunk 0, whose token rows the walks read as
// zeros. Every buffer term is linear in B and lies in chunk 0 (the later chunks see it through the
// state), so the walks keep their chunk code and take these terms from three small launches:
//
//   k_buf_state (before the walks), from the forward chunk's coefficient record:
//     dS_end = -sum_s Ws[s, end] B_s,  dZ_end = sum_s Wz[s, end] B_s, the same after token Lmid - 1
//     (the saved backward-chunk boundary), Z terms only with momentum. k_walk_full adds them to the
//     states after chunk 0; carried through segment 0's later chunks (their end scalars a, kappa, b)
//     the end terms are added to segment 0's aggregate by the segment scan.
//   k_buf_y (after k_walk_full), with the forward chunk's Ws block:
//     y_t += -sum_s Ws[s, t-1] B_s psi_t                                             (t < 64)
//   k_buf_bwd (after k_walk_bwd, before the scalar chain), with the backward chunk's records and the
//   chunk-0 end adjoint (dS_e, dZ_e) the reverse walk leaves in buf_adj:
//     d buffer_in[s] = Wz[s, end] dZ_e - Ws[s, end] dS_e - sum_q Ws[s, q-1] dy_q psi_q^T
//     records of chunk 0: hS[s] += <dS_e, B_s>, hZ[s] += <dZ_e, B_s>, Lm[q][s] += dy_q^T B_s psi_q
//     dq[q] += -(sum_s Ws[s, q-1] B_s^T dy_q) * map'(q)                             (q < 32)
//   (the same terms as the general kernels' first-chunk buffer code, seg_fwd.h / seg_bwd.hip).
// The products run on fp32 matrix cores (v_mfma_f32_16x16x4_f32, mem_common.h's NT convention) with
// the operands staged in LDS as fp32; y and dq are read, corrected and rounded to bf16 again.
#include "mem_common.h"
#include "mem_params.h"
#include "seg_common.h"

#include <algorithm>

namespace atlas {

namespace {

constexpr int kBwThreads = 256;
constexpr int D = bufw::D;
constexpr int P = D + 1;   // LDS pitch of the fp32 operand rows

typedef MM<float> MF;

template <int CH>
struct RecOff {
  static constexpr int SPM = CoefRec<CH>::SPM;
  static constexpr int ACOEF = 0, KCOEF = CH, ENDC = 2 * CH, WSEND = 2 * CH + 4, WZEND = WSEND + SPM,
                       WSMID = WZEND + SPM, WZMID = WSMID + SPM;
};

__device__ __forceinline__ float bf16f(bf16 x) { return static_cast<float>(x); }

// rows [0, n) of D bf16 values (row r at src + r * D) -> dst[r][*] fp32, mapped; rows n .. nr - 1 zero
__device__ __forceinline__ void stage_rows(float (*dst)[P], const bf16* src, int n, int nr, int map_mode, int deg) {
  for (int v = threadIdx.x; v < nr * (D / 8); v += kBwThreads) {
    const int r = v / (D / 8), c = (v % (D / 8)) * 8;
    float x[8];
    if (r < n) {
      const uint4 w = *reinterpret_cast<const uint4*>(src + (size_t)r * D + c);
      const unsigned u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        x[2 * h] = __builtin_bit_cast(float, u[h] << 16);
        x[2 * h + 1] = __builtin_bit_cast(float, u[h] & 0xffff0000u);
      }
      if (map_mode == MAP_ELEMENTWISE) {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = poly_map(x[e], deg);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) dst[r][c + e] = x[e];
  }
}

// one buffer slot [D][D] fp32 -> dst (pitch P)
__device__ __forceinline__ void stage_slot(float (*dst)[P], const float* Bs) {
  for (int v = threadIdx.x; v < D * D / 4; v += kBwThreads) {
    const float4 x = reinterpret_cast<const float4*>(Bs)[v];
    const int i = (4 * v) / D, k = (4 * v) % D;
    dst[i][k] = x.x; dst[i][k + 1] = x.y; dst[i][k + 2] = x.z; dst[i][k + 3] = x.w;
  }
}

// A product's k order is free as long as both operands follow it: the products below give lane
// group kq = lane >> 4 the k values 16 kq + j at step j (16 steps over D = 64), so that a lane's
// operand values are 16 consecutive floats of one row.

// The end scalars (a, kappa, b) of a run of chunks composed in order, later o earlier:
// (a2 a1, a2 k1 + k2 b1, b2 b1).
struct Akb {
  float a, k, b;
};
__device__ __forceinline__ Akb compose(const Akb& later, const Akb& earlier) {
  return Akb{later.a * earlier.a, later.a * earlier.k + later.k * earlier.b, later.b * earlier.b};
}

// grid (D * D / kBwThreads, BH), one state element per thread. G0: the chunks of segment 0 when
// there are several segments (its aggregate gets the end terms carried through chunks 1 .. G0 - 1),
// else 0.
__global__ __launch_bounds__(kBwThreads) void k_buf_state(const Geom g, const FwdPtrs<bf16> a,
                                                          const float* __restrict__ coef, float* __restrict__ corr,
                                                          int G0) {
  if (geom_skip(g)) return;
  constexpr int CH = bufw::CHF;
  using R = RecOff<CH>;
  __shared__ Akb part[kBwThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, bh = blockIdx.y;
  const int idx = blockIdx.x * kBwThreads + tid;
  const int H = g.H;
  const float* rec = coef + (size_t)bh * g.nc * CoefRec<CH>::SIZE;   // chunk 0
  float* out = corr + (size_t)bh * bufw::kCorrFloats;
  const float* Bb = a.buf_in + (size_t)bh * H * D * D + idx;
  float se = 0.f, ze = 0.f, sm = 0.f, zm = 0.f;
  for (int s = 0; s < H; ++s) {
    const float b = Bb[(size_t)s * D * D];
    se -= rec[R::WSEND + s] * b;
    ze += rec[R::WZEND + s] * b;
    sm -= rec[R::WSMID + s] * b;
    zm += rec[R::WZMID + s] * b;
  }
  const float zk = g.momentum ? 1.f : 0.f;
  // chunks 1 .. G0 - 1 with no input: each thread composes its run, then each wave its lanes' (a
  // tree in chunk order) and one thread the four waves'
  const int nrun = G0 > 1 ? (G0 - 1 + kBwThreads - 1) / kBwThreads : 0;
  Akb x{1.f, 0.f, 1.f};
  for (int j = 0; j < nrun; ++j) {
    const int c = 1 + tid * nrun + j;
    if (c < G0) {
      const float* rc = rec + (size_t)c * CoefRec<CH>::SIZE;
      x = compose(Akb{rc[R::ENDC], rc[R::ENDC + 1], zk * rc[R::ENDC + 2]}, x);
    }
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const Akb y{__shfl_down(x.a, o, 64), __shfl_down(x.k, o, 64), __shfl_down(x.b, o, 64)};
    if ((lane & (2 * o - 1)) == 0 && lane + o < 64) x = compose(y, x);
  }
  if (lane == 0) part[tid >> 6] = x;
  __syncthreads();
  Akb t = part[0];
#pragma unroll
  for (int w = 1; w < kBwThreads / 64; ++w) t = compose(part[w], t);
  out[bufw::SE + idx] = se;
  out[bufw::ZE + idx] = zk * ze;
  out[bufw::SM + idx] = sm;
  out[bufw::ZM + idx] = zk * zm;
  out[bufw::AU + idx] = t.a * se - t.k * zk * ze;
  out[bufw::AV + idx] = zk * t.b * ze;
}

// grid (CHF / 16, BH): workgroup x corrects y of tokens 16 x .. 16 x + 15, wave w rows 16 w ..:
//   Y[i][t] = -sum_s sum_k B_s[i][k] (Ws[s, t-1] psi_t[k])   (one product over K = (e-1) * D)
__global__ __launch_bounds__(kBwThreads) void k_buf_y(const Geom g, const FwdPtrs<bf16> a, const bf16* __restrict__ wsh) {
  if (geom_skip(g)) return;
  constexpr int CH = bufw::CHF, TG = 16;
  using R = RecOff<CH>;
  __shared__ float sps[TG][P];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, bh = blockIdx.y, t0 = blockIdx.x * TG;
  const int H = g.H, L = min(g.T, CH);
  if (t0 >= L) return;   // workgroup-uniform
  const bf16* w0 = wsh + (size_t)bh * g.nc * CH * R::SPM;   // chunk 0: Ws rows [t][s]
  stage_rows(sps, a.q + ((size_t)bh * g.T + t0) * D, min(TG, L - t0), TG, g.map_mode, g.map_deg);
  __syncthreads();
  const int tl = lane & 15, kq = lane >> 4;
  // A = B_s rows 16 w + tl straight from memory: 16 consecutive k per lane
  const float* Brow = a.buf_in + ((size_t)bh * H * D + 16 * w + tl) * D + 16 * kq;
  f32x4 acc = zero4();
  for (int s = 0; s < H; ++s) {
    float4 bv[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) bv[v] = reinterpret_cast<const float4*>(Brow + (size_t)s * D * D)[v];
    const float wt = t0 + tl < L ? bf16f(w0[(size_t)(t0 + tl) * R::SPM + s]) : 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float bb[4] = {bv[v].x, bv[v].y, bv[v].z, bv[v].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = MF::mma(bb[e], wt * sps[tl][16 * kq + 4 * v + e], acc);
    }
  }
  // the accumulator is read after the loop's exit: one unconditional (zero) product first, so that
  // the read never follows a join directly after an MFMA that was issued conditionally
  acc = MF::mma(0.f, 0.f, acc);
  // lane: rows 16 w + 4 kq + r of token t0 + tl
  const int t = t0 + tl;
  if (t < L) {
    bf16* yp = a.y + ((size_t)bh * g.T + t) * D + 16 * w + 4 * kq;
#pragma unroll
    for (int r = 0; r < 4; ++r) yp[r] = from_f32<bf16>(bf16f(yp[r]) - acc[r]);
  }
}

// grid (e, BH): workgroup s < e - 1 forms d buffer_in[s] and slot s's record terms; workgroup e - 1
// the dq terms of the first backward chunk (every slot).
__global__ __launch_bounds__(kBwThreads) void k_buf_bwd(const Geom g, const BwdPtrs<bf16> a, const BwdSegPtrs p) {
  if (geom_skip(g)) return;
  constexpr int CH = bufw::CHB;
  using R = RecOff<CH>;
  using SB = ScalarBlock<CH>;
  __shared__ float sB[D][P];
  __shared__ float sdy[CH][P];
  __shared__ float sps[CH][P];
  __shared__ float sw[CH];
  __shared__ float sred[2][kBwThreads / 64];
  __shared__ float slm[2][CH];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, bh = blockIdx.y, s = blockIdx.x;
  const int tl = lane & 15, kq = lane >> 4;
  const int H = g.H, Lq = min(g.T, CH);
  const size_t tb = (size_t)bh * g.T;
  const float* rec = p.coef + (size_t)bh * g.nc * CoefRec<CH>::SIZE;                       // chunk 0
  const bf16* w0 = reinterpret_cast<const bf16*>(p.wsh) + (size_t)bh * g.nc * CH * R::SPM;  // chunk 0
  float* blk = p.scal + (size_t)bh * g.nc * SB::SIZE;                                       // chunk 0
  const float* Bb = a.buf_in + (size_t)bh * H * D * D;
  stage_rows(sdy, a.dy + tb * D, Lq, CH, MAP_OFF, 1);
  if (s == H) {
    // dq: C[k][q] = sum_s sum_i B_s[i][k] (w(q, s) dy_q[i]); wave w: features 16 w .., both token
    // tiles; A[k][i] = B_s[i][k] straight from memory (lane: column 16 w + tl, rows 16 kq + j)
    __syncthreads();   // dy staged
    f32x4 acc[2] = {zero4(), zero4()};
    const float* Bcol = Bb + (size_t)(16 * kq) * D + 16 * w + tl;
    for (int sl = 0; sl < H; ++sl) {
      float bc[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) bc[j] = Bcol[(size_t)sl * D * D + j * D];
      float wq[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) wq[u] = 16 * u + tl < Lq ? bf16f(w0[(size_t)(16 * u + tl) * R::SPM + sl]) : 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j)
#pragma unroll
        for (int u = 0; u < 2; ++u) acc[u] = MF::mma(bc[j], wq[u] * sdy[16 * u + tl][16 * kq + j], acc[u]);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) acc[u] = MF::mma(0.f, 0.f, acc[u]);   // as in k_buf_y: after the loop's exit
    // lane: features 16 w + 4 kq + r of token 16 u + tl
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int q = 16 * u + tl;
      if (q < Lq) {
        const size_t o = (tb + q) * D + 16 * w + 4 * kq;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float mg = g.map_mode == MAP_ELEMENTWISE ? poly_map_grad(bf16f(a.q[o + r]), g.map_deg) : 1.f;
          a.dq[o + r] = from_f32<bf16>(bf16f(a.dq[o + r]) - acc[u][r] * mg);
        }
      }
    }
    return;   // workgroup-uniform
  }
  // slot s: B_s, psi of the chunk's tokens, the weights w(q, s)
  stage_slot(sB, Bb + (size_t)s * D * D);
  stage_rows(sps, a.q + tb * D, Lq, CH, g.map_mode, g.map_deg);
  if (tid < CH) sw[tid] = tid < Lq ? bf16f(w0[(size_t)tid * R::SPM + s]) : 0.f;
  __syncthreads();
  {   // d buffer_in[s] tiles (rows 16 w .., columns 16 j ..): A[i][q] = w(q, s) dy_q[i], Bt[k][q] = psi_q[k]
    const float* dSe = p.buf_adj + (size_t)bh * bufw::kAdjFloats;
    const float* dZe = dSe + D * D;
    const float ws = rec[R::WSEND + s], wz = rec[R::WZEND + s];
    float hs = 0.f, hz = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f32x4 acc = zero4();
#pragma unroll
      for (int jq = 0; jq < CH / 4; ++jq) {   // token q = 8 kq + jq at step jq
        const int q = (CH / 4) * kq + jq;
        acc = MF::mma(sw[q] * sdy[q][16 * w + tl], sps[q][16 * j + tl], acc);
      }
      // lane: rows i = 16 w + 4 kq + r, column k = 16 j + tl
      const int k = 16 * j + tl;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * w + 4 * kq + r;
        const float es = dSe[i * D + k], ez = dZe[i * D + k], b = sB[i][k];
        hs += es * b;
        hz += ez * b;
        a.dbuf_in[(((size_t)bh * H + s) * D + i) * D + k] = wz * ez - ws * es - acc[r];
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      hs += __shfl_xor(hs, off, 64);
      hz += __shfl_xor(hz, off, 64);
    }
    if (lane == 0) { sred[0][w] = hs; sred[1][w] = hz; }
  }
  {   // Lm[q][s] += sum_i dy_q[i] V[i][q], V = B_s psi^T: wave w rows 32 (w >> 1) .. +31, tokens 16 (w & 1) ..
    const int q = 16 * (w & 1) + tl;
    float lm = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int m0 = 32 * (w >> 1) + 16 * h;
      f32x4 acc = zero4();
#pragma unroll
      for (int j = 0; j < 16; ++j) acc = MF::mma(sB[m0 + tl][16 * kq + j], sps[q][16 * kq + j], acc);
      // lane: rows m0 + 4 kq + r of token q
#pragma unroll
      for (int r = 0; r < 4; ++r) lm += sdy[q][m0 + 4 * kq + r] * acc[r];
    }
    lm += __shfl_xor(lm, 16, 64);
    lm += __shfl_xor(lm, 32, 64);
    if (kq == 0) slm[w >> 1][q] = lm;
  }
  __syncthreads();
  if (tid < CH) {
    if (tid < Lq) blk[SB::LM + tid * SB::SPM + s] += slm[0][tid] + slm[1][tid];
  } else if (tid == CH) {
    float hs = 0.f, hz = 0.f;
#pragma unroll
    for (int ww = 0; ww < kBwThreads / 64; ++ww) { hs += sred[0][ww]; hz += sred[1][ww]; }
    blk[SB::HS + s] += hs;
    blk[SB::HZ + s] += hz;
  }
}

}  // namespace

hipError_t launch_buf_state(const Geom& g, const FwdPtrs<bf16>& a, const SegGeom& sg, const float* coef, float* corr,
                            hipStream_t stream) {
  const int G0 = sg.nseg > 1 ? std::min(sg.G, g.nc) : 0;
  prof_name(KID_BUF_FWD, "k_buf_state+k_buf_y");
  prof_begin(KID_BUF_FWD, stream);
  hipLaunchKernelGGL(k_buf_state, dim3(D * D / kBwThreads, g.BH), dim3(kBwThreads), 0, stream, g, a, coef, corr, G0);
  prof_end(KID_BUF_FWD, stream);
  return hipGetLastError();
}

hipError_t launch_buf_y(const Geom& g, const FwdPtrs<bf16>& a, const bf16* wsh, hipStream_t stream) {
  prof_begin(KID_BUF_FWD, stream);
  hipLaunchKernelGGL(k_buf_y, dim3(bufw::CHF / 16, g.BH), dim3(kBwThreads), 0, stream, g, a, wsh);
  prof_end(KID_BUF_FWD, stream);
  return hipGetLastError();
}

hipError_t launch_buf_bwd(const Geom& g, const BwdPtrs<bf16>& a, const BwdSegPtrs& p, hipStream_t stream) {
  prof_name(KID_BUF_BWD, "k_buf_bwd");
  prof_begin(KID_BUF_BWD, stream);
  hipLaunchKernelGGL(k_buf_bwd, dim3(g.e, g.BH), dim3(kBwThreads), 0, stream, g, a, p);
  prof_end(KID_BUF_BWD, stream);
  return hipGetLastError();
}

}  // namespace atlas
