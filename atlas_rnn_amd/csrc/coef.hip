// coef.hip - per-chunk coefficients of the chunked closed form, for every chunk of every row.
//
// The coefficients of a chunk depend only on its decay / lr / beta / gate values, never on the
// states, so they are formed here ahead of the segment walks, with one small thread group per
// (chunk, bh) and many workgroups per CU: the step-by-step recurrences that would otherwise sit on
// a walk's critical path overlap across chunks. One launch in the forward forms the records of
// the forward chunks and of the backward chunks (k_chunk_coef_pair). Per chunk:
//   record (fp32): acoef[CH] = a_{t-1}, kcoef[CH] = kappa_{t-1}, endc = (a, kappa, b) of the chunk,
//                  wsend[SPM] = Ws[s, end], wzend[SPM] = Wz[s, end]
//   wsh (T):       Ws[s, t-1] as [CH][SPM] (optional)
// The walks prefetch these with the chunk's other inputs.
#include "mem_common.h"
#include "mem_params.h"
#include "seg_common.h"
#include "walk_common.h"

namespace atlas {

// One lane per source (sources 0 .. SPM-1, SPM = CH + 32), rounded up to whole waves.
template <int CH>
constexpr int coef_threads() { return (CH + kHaloPad + 63) / 64 * 64; }

template <int CH>
struct CoefSmem {
  static constexpr int SPM = CH + kHaloPad;
  alignas(16) float alpha[CH];   // padded steps: alpha = beta = 1, eta = 0
  alignas(16) float eta[CH];
  alignas(16) float beta[CH];
  // [t][s]: the window weight w(s, t) (zero outside the window) until lane s reads it, then
  // Ws[s, t-1] (each lane reads and overwrites only its own column, in order)
  alignas(16) float tab[CH][SPM];
};

// Record layout (floats): acoef[CH], kcoef[CH], endc[4], wsend[SPM], wzend[SPM], wsmid[SPM],
// wzmid[SPM], midc[4].
//   source s:   Wz[s,t] = beta_t Wz[s,t-1] + w(s,t),  Ws[s,t] = alpha_t Ws[s,t-1] + eta_t Wz[s,t]
//               one lane per source, three VALU operations and two LDS accesses per step; Ws[s, t-1]
//               goes to the table and from there, after the chains, to wsh[t][s] in 16-byte stores;
//   prefix:     when H + CH <= SPM - 2 (e <= 31), the two last source lanes never see a window
//               weight and run the same chain from Ws = 1 (lane SPM-2: Ws_t = a_t = prod alpha) and
//               from Wz = 1 (lane SPM-1: Wz_t = b_t = prod beta, Ws_t = kappa_t); acoef and kcoef
//               are their table columns. Otherwise inclusive scans across the last wave's lanes.
//   mid values: after token Lmid - 1 (a multiple of 8) when Lmid > 0, else zero.
// The inputs (step scalars, and the gates of windows up to 4 NT / CH) are loaded together, ahead
// of the first barrier.
// Chunk c of row bh, by coef_threads<CH>() threads (tid) with the LDS block sm. Every thread of
// the workgroup reaches the same barriers, whichever chunk (and chunk length) its group works on.
// HALF: the chunk's first half is a backward chunk of its own (Lmid = CH / 2, the backward's
// chunk); its record is the forward record's values at the mid point and its Ws block the first
// CH / 2 rows of the forward table, written to rec_h / wsh_h (backward chunk 2c of geometry gh).
// Used only when both prefix-lane conditions hold (see k_chunk_coef_pair).
template <typename T, int CH, bool WSH, bool HALF = false>
__device__ __forceinline__ void chunk_coef(const Geom& g, const T* __restrict__ decay, const T* __restrict__ lr,
                                           const T* __restrict__ beta, const T* __restrict__ gate,
                                           float* __restrict__ rec_all, T* __restrict__ wsh, int c, int bh, int tid,
                                           CoefSmem<CH>& sm, const Geom* gh = nullptr,
                                           float* __restrict__ rec_h_all = nullptr, T* __restrict__ wsh_h = nullptr) {
  constexpr int CHH = CH / 2, SPMH = CHH + kHaloPad, RECH = CoefRec<CHH>::SIZE;
  constexpr int H_KCOEF = CHH, H_ENDC = 2 * CHH, H_WSEND = H_ENDC + 4, H_WZEND = H_WSEND + SPMH,
                H_WSMID = H_WZEND + SPMH, H_WZMID = H_WSMID + SPMH, H_MIDC = H_WZMID + SPMH;
  constexpr int SPM = CH + kHaloPad, NT = coef_threads<CH>(), REC = CoefRec<CH>::SIZE;
  constexpr int R_KCOEF = CH, R_ENDC = 2 * CH, R_WSEND = R_ENDC + 4, R_WZEND = R_WSEND + SPM,
                R_WSMID = R_WZEND + SPM, R_WZMID = R_WSMID + SPM, R_MIDC = R_WZMID + SPM;
  constexpr int GRP = NT / CH, JR = 4;   // threads per target; gates held per thread
  constexpr int LA = SPM - 2, LK = SPM - 1;   // prefix lanes
  static_assert(R_MIDC + 4 == REC, "record layout");
  static_assert(CH <= 64 && (CH & (CH - 1)) == 0 && CH % 8 == 0 && NT % CH == 0 && SPM % 8 == 0, "lanes");
  const int lane = tid & 63;
  const int H = g.H, e = g.e;
  const int t0 = c * g.Lc, L = min(g.T, t0 + g.Lc) - t0;
  const size_t tb = (size_t)bh * g.T, r0 = tb + t0;
  float* rec = rec_all + ((size_t)bh * g.nc + c) * REC;
  const bool scan_wave = tid >= NT - 64;            // wave-uniform
  const bool lane_prefix = H + CH <= SPM - 2;       // uniform
  const bool few_gates = e <= JR * GRP;             // uniform

  // ---- inputs: step scalars (last wave, lane t), window weights of target tt, lags jg + GRP r
  float al = 1.f, et = 0.f, be = 1.f;
  {   // every lane loads (clamped index, no branch around the loads); the last wave's lanes t < L keep them
    const size_t rt = r0 + min(lane, L - 1);
    const T xa = decay[rt], xe = lr[rt], xb = (g.momentum && beta ? beta : decay)[rt];
    const bool keep = scan_wave && lane < min(CH, L);
    const float fa = to_f32(xa), fe = to_f32(xe), fb = g.momentum ? to_f32(xb) : 0.f;
    al = keep ? fa : 1.f;
    et = keep ? fe : 0.f;
    be = keep ? fb : 1.f;
  }
  const int tt = tid % CH, jg = tid / CH;
  auto weight = [&](int j) {   // w(tt + H - j, tt); the load is issued for any j, tt (clamped index)
    const int tc = min(tt, L - 1), jc = min(j, e - 1);
    if (g.gate_mode == GATE_LAG) return to_f32(gate[(r0 + tc) * e + jc]);
    if (g.gate_mode == GATE_TOKEN) {
      const int p = t0 + tc - jc;   // source token
      const float x = to_f32(gate[tb + (p >= 0 ? p : 0)]);
      return p >= 0 ? x : 1.f;
    }
    return 1.f;
  };
  float gv[JR];
  if (few_gates) {   // one uniform branch around all JR loads, so that they are in flight together
    T raw[JR];
    if (g.gate_mode == GATE_LAG) {
#pragma unroll
      for (int r = 0; r < JR; ++r) {
        const int tc = min(tt, L - 1), jc = min(jg + GRP * r, e - 1);
        raw[r] = gate[(r0 + tc) * e + jc];
      }
#pragma unroll
      for (int r = 0; r < JR; ++r) gv[r] = to_f32(raw[r]);
    } else if (g.gate_mode == GATE_TOKEN) {
#pragma unroll
      for (int r = 0; r < JR; ++r) {
        const int p = t0 + min(tt, L - 1) - min(jg + GRP * r, e - 1);
        raw[r] = gate[tb + (p >= 0 ? p : 0)];
      }
#pragma unroll
      for (int r = 0; r < JR; ++r) {
        const int p = t0 + min(tt, L - 1) - min(jg + GRP * r, e - 1);
        gv[r] = p >= 0 ? to_f32(raw[r]) : 1.f;
      }
    } else {
#pragma unroll
      for (int r = 0; r < JR; ++r) gv[r] = 1.f;
    }
  }
  for (int i = tid; i < CH * SPM / 4; i += NT)
    reinterpret_cast<float4*>(&sm.tab[0][0])[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  if (scan_wave && lane < CH) {
    sm.alpha[lane] = al;
    sm.eta[lane] = et;
    sm.beta[lane] = be;
  }
  __syncthreads();
  if (tt < L) {   // target tt, lag j -> source s = tt + H - j (0 .. SPM-1 since H = e - 1 <= 32)
    if (few_gates) {
#pragma unroll
      for (int r = 0; r < JR; ++r) {
        const int j = jg + GRP * r;
        if (j < e) sm.tab[tt][tt + H - j] = gv[r];
      }
    } else {
      for (int j = jg; j < e; j += GRP) sm.tab[tt][tt + H - j] = weight(j);
    }
  }
  __syncthreads();

  if (!lane_prefix && scan_wave) {   // prefix coefficients by scans, lane t = step t
    float b = be;
#pragma unroll
    for (int d = 1; d < CH; d <<= 1) {
      const float o = __shfl_up(b, d, 64);
      if (lane >= d) b *= o;
    }
    float A = al, K = et * b;   // (A, K) o (A', K') = (A A', A K' + K)
#pragma unroll
    for (int d = 1; d < CH; d <<= 1) {
      const float oA = __shfl_up(A, d, 64), oK = __shfl_up(K, d, 64);
      if (lane >= d) {
        K = fmaf(A, oK, K);
        A *= oA;
      }
    }
    const float ap = __shfl_up(A, 1, 64), kp = __shfl_up(K, 1, 64);
    if (lane < CH) {
      rec[lane] = lane ? ap : 1.f;
      rec[R_KCOEF + lane] = lane ? kp : 0.f;
    }
    if (lane == CH - 1) *reinterpret_cast<float4*>(rec + R_ENDC) = make_float4(A, K, b, 0.f);
    if (g.Lmid > 0 ? lane == g.Lmid - 1 : lane == 0)
      *reinterpret_cast<float4*>(rec + R_MIDC) = g.Lmid > 0 ? make_float4(A, K, b, 0.f) : make_float4(0.f, 0.f, 0.f, 0.f);
  }

  if (tid < SPM) {   // chains
    const int s = tid;
    float ws = (lane_prefix && s == LA) ? 1.f : 0.f, wz = (lane_prefix && s == LK) ? 1.f : 0.f;
    float wsm = 0.f, wzm = 0.f;
#pragma unroll
    for (int t8 = 0; t8 < CH; t8 += 8) {
      float a8[8], e8[8], b8[8], w8[8];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float4 xa = *reinterpret_cast<const float4*>(&sm.alpha[t8 + 4 * h]);
        const float4 xe = *reinterpret_cast<const float4*>(&sm.eta[t8 + 4 * h]);
        const float4 xb = *reinterpret_cast<const float4*>(&sm.beta[t8 + 4 * h]);
        a8[4 * h] = xa.x; a8[4 * h + 1] = xa.y; a8[4 * h + 2] = xa.z; a8[4 * h + 3] = xa.w;
        e8[4 * h] = xe.x; e8[4 * h + 1] = xe.y; e8[4 * h + 2] = xe.z; e8[4 * h + 3] = xe.w;
        b8[4 * h] = xb.x; b8[4 * h + 1] = xb.y; b8[4 * h + 2] = xb.z; b8[4 * h + 3] = xb.w;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) w8[u] = sm.tab[t8 + u][s];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        sm.tab[t8 + u][s] = ws;   // Ws[s, t-1]
        wz = fmaf(b8[u], wz, w8[u]);
        ws = fmaf(a8[u], ws, e8[u] * wz);
      }
      if (t8 + 8 == g.Lmid) {   // wave-uniform
        wsm = ws;
        wzm = wz;
      }
    }
    const bool src = !(lane_prefix && s >= LA);
    rec[R_WSEND + s] = src ? ws : 0.f;
    rec[R_WZEND + s] = src ? wz : 0.f;
    rec[R_WSMID + s] = src ? wsm : 0.f;
    rec[R_WZMID + s] = src ? wzm : 0.f;
    if constexpr (HALF) {   // the half's sources are the first SPMH; its own prefix columns stay zero
      float* rh = rec_h_all + ((size_t)bh * gh->nc + 2 * c) * RECH;
      if (s < SPMH) {
        const bool hs = s < SPMH - 2;
        rh[H_WSEND + s] = hs ? wsm : 0.f;
        rh[H_WZEND + s] = hs ? wzm : 0.f;
        rh[H_WSMID + s] = 0.f;
        rh[H_WZMID + s] = 0.f;
      }
      if (s == LA) *reinterpret_cast<float4*>(rh + H_MIDC) = make_float4(0.f, 0.f, 0.f, 0.f);
      if (s == LA) rh[H_ENDC] = wsm;
      if (s == LK) { rh[H_ENDC + 1] = wsm; rh[H_ENDC + 2] = wzm; rh[H_ENDC + 3] = 0.f; }
    }
    if (!src) {   // (a, kappa, b) at the end and after token Lmid - 1
      if (s == LA) {
        rec[R_ENDC] = ws;
        rec[R_MIDC] = wsm;
      } else {
        rec[R_ENDC + 1] = ws;
        rec[R_ENDC + 2] = wz;
        rec[R_ENDC + 3] = 0.f;
        rec[R_MIDC + 1] = wsm;
        rec[R_MIDC + 2] = wzm;
        rec[R_MIDC + 3] = 0.f;
      }
    }
  }
  __syncthreads();

  if (lane_prefix && tid < CH) {   // acoef = a_{t-1}, kcoef = kappa_{t-1}
    rec[tid] = sm.tab[tid][LA];
    rec[R_KCOEF + tid] = sm.tab[tid][LK];
  }
  if constexpr (HALF) {
    float* rh = rec_h_all + ((size_t)bh * gh->nc + 2 * c) * RECH;
    if (tid < CHH) {
      rh[tid] = sm.tab[tid][LA];
      rh[H_KCOEF + tid] = sm.tab[tid][LK];
    }
    // Ws block of the half: table rows t < CHH, sources s < SPMH (its prefix columns zeroed)
    const rsrc_t rw = make_rsrc(wsh_h + ((size_t)bh * gh->nc + 2 * c) * CHH * SPMH, (uint32_t)(CHH * SPMH * sizeof(T)));
    constexpr int G8 = SPMH / 8;
    for (int i = tid; i < CHH * G8; i += NT) {
      const int t = i / G8, s0 = (i % G8) * 8;
      float v[8];
      const float4 x0 = *reinterpret_cast<const float4*>(&sm.tab[t][s0]);
      const float4 x1 = *reinterpret_cast<const float4*>(&sm.tab[t][s0 + 4]);
      v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w; v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
      if (s0 == SPMH - 8) { v[6] = 0.f; v[7] = 0.f; }
      const uint32_t off = (uint32_t)((t * SPMH + s0) * sizeof(T));
      if constexpr (sizeof(T) == 2) {
        u32x4v o;
        o[0] = pack_bf16x2(v[0], v[1]);
        o[1] = pack_bf16x2(v[2], v[3]);
        o[2] = pack_bf16x2(v[4], v[5]);
        o[3] = pack_bf16x2(v[6], v[7]);
        bst16(rw, off, o);
      } else {
        const u32x4v o0 = {__builtin_bit_cast(unsigned, v[0]), __builtin_bit_cast(unsigned, v[1]),
                           __builtin_bit_cast(unsigned, v[2]), __builtin_bit_cast(unsigned, v[3])};
        const u32x4v o1 = {__builtin_bit_cast(unsigned, v[4]), __builtin_bit_cast(unsigned, v[5]),
                           __builtin_bit_cast(unsigned, v[6]), __builtin_bit_cast(unsigned, v[7])};
        bst16(rw, off, o0);
        bst16(rw, off + 16, o1);
      }
    }
  }
  if constexpr (WSH) {   // Ws[s, t-1] -> wsh[t][s], eight sources per store (prefix columns zeroed)
    const rsrc_t rw = make_rsrc(wsh + ((size_t)bh * g.nc + c) * CH * SPM, (uint32_t)(CH * SPM * sizeof(T)));
    constexpr int G8 = SPM / 8;
    for (int i = tid; i < CH * G8; i += NT) {
      const int t = i / G8, s0 = (i % G8) * 8;
      float v[8];
      const float4 x0 = *reinterpret_cast<const float4*>(&sm.tab[t][s0]);
      const float4 x1 = *reinterpret_cast<const float4*>(&sm.tab[t][s0 + 4]);
      v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w; v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
      if (lane_prefix && s0 == SPM - 8) { v[6] = 0.f; v[7] = 0.f; }
      const uint32_t off = (uint32_t)((t * SPM + s0) * sizeof(T));
      if constexpr (sizeof(T) == 2) {
        u32x4v o;
        o[0] = pack_bf16x2(v[0], v[1]);
        o[1] = pack_bf16x2(v[2], v[3]);
        o[2] = pack_bf16x2(v[4], v[5]);
        o[3] = pack_bf16x2(v[6], v[7]);
        bst16(rw, off, o);
      } else {
        const u32x4v o0 = {__builtin_bit_cast(unsigned, v[0]), __builtin_bit_cast(unsigned, v[1]),
                           __builtin_bit_cast(unsigned, v[2]), __builtin_bit_cast(unsigned, v[3])};
        const u32x4v o1 = {__builtin_bit_cast(unsigned, v[4]), __builtin_bit_cast(unsigned, v[5]),
                           __builtin_bit_cast(unsigned, v[6]), __builtin_bit_cast(unsigned, v[7])};
        bst16(rw, off, o0);
        bst16(rw, off + 16, o1);
      }
    }
  }
}

// Forward (CHF) and backward (CHB) chunk records in one launch: workgroups x < gf.nc form forward
// chunks, the others PER backward chunks each (one thread group per chunk; a group past the last
// chunk repeats it, writing the same values). Both depend only on the per-token scalars.
template <typename T, int CHF, int CHB>
__global__ __launch_bounds__(coef_threads<CHF>()) void k_chunk_coef_pair(
    const Geom gf, const Geom gb, const T* __restrict__ decay, const T* __restrict__ lr, const T* __restrict__ beta,
    const T* __restrict__ gate, float* __restrict__ rec_f, T* __restrict__ wsh_f, float* __restrict__ rec_b,
    T* __restrict__ wsh_b, int halves) {
  if (geom_skip(gf)) return;
  if (gf.flag_reset && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *const_cast<int*>(gf.flag) = 0;
  constexpr int NTB = coef_threads<CHB>(), PER = coef_threads<CHF>() / NTB;
  static_assert(coef_threads<CHF>() % NTB == 0, "backward groups per workgroup");
  __shared__ union U {
    CoefSmem<CHF> f;
    CoefSmem<CHB> b[PER];
  } sm;
  const int x = blockIdx.x, bh = blockIdx.y;
  if (x < gf.nc) {
    if (halves)
      chunk_coef<T, CHF, true, true>(gf, decay, lr, beta, gate, rec_f, wsh_f, x, bh, threadIdx.x, sm.f, &gb, rec_b,
                                     wsh_b);
    else
      chunk_coef<T, CHF, true>(gf, decay, lr, beta, gate, rec_f, wsh_f, x, bh, threadIdx.x, sm.f);
  } else {
    const int j = threadIdx.x / NTB;
    const int i = (x - gf.nc) * PER + j;   // backward chunk i, or odd chunk 2 i + 1 when halves
    const int c = halves ? min(2 * i + 1, gb.nc - 1 - (gb.nc % 2 == 1)) : min(i, gb.nc - 1);
    chunk_coef<T, CHB, true>(gb, decay, lr, beta, gate, rec_b, wsh_b, c, bh, threadIdx.x % NTB, sm.b[j]);
  }
}

// Whether the forward chunks' first halves give the even backward chunks (k_chunk_coef_pair).
template <int CHF, int CHB>
bool coef_halves(const Geom& gf, const Geom& gb) {
  return CHF == 2 * CHB && gb.Lc == CHB && gf.Lc == CHF && gf.Lmid == CHB && gf.H + CHF <= CHF + kHaloPad - 2 &&
         gb.H + CHB <= CHB + kHaloPad - 2;
}

template <typename T, int CHF, int CHB>
hipError_t launch_chunk_coef_pair(const Geom& gf, const Geom& gb, const T* decay, const T* lr, const T* beta,
                                  const T* gate, float* rec_f, T* wsh_f, float* rec_b, T* wsh_b, hipStream_t stream) {
  if (gf.Lmid % 8 != 0 || gf.Lmid > CHF || gb.Lmid != 0) return hipErrorInvalidValue;
  constexpr int PER = coef_threads<CHF>() / coef_threads<CHB>();
  // rec_b null: the forward records only (a backward that forms its coefficients itself)
  const int halves = rec_b && coef_halves<CHF, CHB>(gf, gb) ? 1 : 0;
  const int nb = !rec_b ? 0 : halves ? gb.nc / 2 : gb.nc;   // backward chunks formed by their own thread groups
  prof_name(KID_FWD_COEF, "k_chunk_coef_pair");
  prof_begin(KID_FWD_COEF, stream);
  hipLaunchKernelGGL((k_chunk_coef_pair<T, CHF, CHB>), dim3(gf.nc + (nb + PER - 1) / PER, gf.BH),
                     dim3(coef_threads<CHF>()), 0, stream, gf, gb, decay, lr, beta, gate, rec_f, wsh_f, rec_b, wsh_b,
                     halves);
  prof_end(KID_FWD_COEF, stream);
  return hipGetLastError();
}

template hipError_t launch_chunk_coef_pair<bf16, 64, 32>(const Geom&, const Geom&, const bf16*, const bf16*, const bf16*,
                                                         const bf16*, float*, bf16*, float*, bf16*, hipStream_t);
template hipError_t launch_chunk_coef_pair<float, 32, 16>(const Geom&, const Geom&, const float*, const float*,
                                                          const float*, const float*, float*, float*, float*, float*,
                                                          hipStream_t);

}  // namespace atlas
