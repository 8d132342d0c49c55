// seg_fixup.h - segment-boundary fixup of the backward pass, shared by k_bwd_seg_fixup (seg_bwd.hip)
// and the scalar-gradient launch of the specialised path (walk_bwd.hip), which runs it as extra
// workgroups beside the scalar chains when the two do not depend on each other.
//
// Workgroup (seg, bh), kThreads threads: merges the partial (dv, dphi) of the tokens whose window
// crosses the segment's end (its tail record and the next segment's halo record), forms the
// token-gate gradients of its tokens, and (reduce_dsref) sums its share of the dS_ref partials over
// the segments. OUTBUF = false leaves out the d buffer_out terms (no buffer_out gradient given).
#pragma once

#include "mem_common.h"
#include "mem_params.h"
#include "seg_common.h"

namespace atlas {

template <typename T, int D, bool OUTBUF>
__device__ __forceinline__ void bwd_seg_fixup(const Geom& g, const BwdPtrs<T>& a, const SegGeom& sg,
                                              const BwdSegPtrs& p, int reduce_dsref, int seg, int bh) {
  __shared__ float sphi[D], sdel[D], sdd[D], sdb[D];
  const int H = g.H, e = g.e;
  const int c_begin = seg * sg.G, c_end = min(g.nc, c_begin + sg.G);
  const int tok0 = c_begin * g.Lc, tok1 = min(g.T, c_end * g.Lc);
  const size_t tb = (size_t)bh * g.T;
  const int tid = threadIdx.x;
  auto reduce = [&]() {
    if (!reduce_dsref) return;
    const int per = (D * D + sg.nseg - 1) / sg.nseg;
    const int i0 = seg * per, i1 = min(D * D, i0 + per);
    const float* part = p.dsref_part + (size_t)bh * sg.nseg * D * D;
    for (int idx = i0 + tid; idx < i1; idx += kThreads) {
      float acc = 0.f;
      for (int s0 = 0; s0 < sg.nseg; s0 += 8) {   // eight partials per memory round trip
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = part[(size_t)min(s0 + u, sg.nseg - 1) * D * D + idx];
#pragma unroll
        for (int u = 0; u < 8; ++u) acc += s0 + u < sg.nseg ? v[u] : 0.f;
      }
      a.dS_ref[(size_t)bh * D * D + idx] = acc;
    }
  };
  constexpr int HF = 16;   // tail tokens of the single-round-trip pass
  const bool fast = (!OUTBUF || a.dbuf_out == nullptr) && g.H > 0 && g.H <= HF;
  if (!fast) reduce();
  // token-gate gradient du_p = sum_j dw[p + j, j] (the d buffer_out term is added below)
  if (g.gate_mode == GATE_TOKEN) {
    for (int pp = tok0 + tid; pp < tok1; pp += kThreads) {
      if (a.dbuf_out && pp >= g.T - H) continue;
      float du = 0.f;
      for (int j = 0; j < e && pp + j < g.T; ++j) du += p.dw[(tb + pp + j) * e + j];
      a.dgate[tb + pp] = from_f32<T>(du);
    }
  }
  if (H == 0) return;
  const int tail0 = tok1 - H;
  const bool has_next = seg + 1 < sg.nseg;
  if (fast) {
    // no buffer_out terms: the 2 D values of each tail token are independent sums of two partials;
    // their loads are issued before the dS_ref sum's, so that the launch waits for one round trip
    constexpr int NV = (2 * HF * D + kThreads - 1) / kThreads;
    float val[NV];
    int dst[NV];
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      dst[u] = -1;
      val[u] = 0.f;
      if (u * kThreads >= H * 2 * D) continue;   // uniform
      const int idx = tid + u * kThreads;
      const int h = idx / (2 * D), col = idx % (2 * D);
      const int pp = tail0 + h;
      const bool ok = h < H && pp >= tok0;   // (a token before tok0 belongs to the previous segment)
      const size_t tp = (((size_t)bh * sg.nseg + seg) * H + (ok ? h : 0)) * (2 * D);
      const size_t hp = (((size_t)bh * sg.nseg + seg + (has_next ? 1 : 0)) * H + (ok ? h : 0)) * (2 * D);
      const float tv = p.tail_part[tp + col], hv = p.halo_part[hp + col];   // in range for every lane
      val[u] = ok ? tv + (has_next ? hv : 0.f) : 0.f;
      dst[u] = ok ? col : -1;
    }
    reduce();
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      if (dst[u] < 0) continue;
      const int idx = tid + u * kThreads, pp = tail0 + idx / (2 * D), col = dst[u];
      if (col < D) {
        a.dv[(tb + pp) * D + col] = from_f32<T>(val[u]);
      } else {
        float v = val[u];
        if (g.map_mode == MAP_ELEMENTWISE) v *= poly_map_grad(to_f32(a.k[(tb + pp) * D + col - D]), g.map_deg);
        a.dk[(tb + pp) * D + col - D] = from_f32<T>(v);
      }
    }
    return;
  }
  for (int h = 0; h < H; ++h) {
    const int pp = tail0 + h;
    if (pp < tok0) continue;                       // token of the previous segment (short last segment)
    const size_t tp = (((size_t)bh * sg.nseg + seg) * H + h) * (2 * D);
    const size_t hp = has_next ? (((size_t)bh * sg.nseg + seg + 1) * H + h) * (2 * D) : 0;
    const bool outbuf = OUTBUF && (a.dbuf_out != nullptr) && (pp >= g.T - H);
    const int kb = pp - (g.T - H);
    __syncthreads();
    if (outbuf) {
      for (int k = tid; k < D; k += kThreads) sphi[k] = ld_map(a.k, (tb + pp) * D + k, g.map_mode, g.map_deg);
      __syncthreads();
      const float cp = (g.gate_mode == GATE_TOKEN) ? to_f32(a.gate[tb + pp]) : 1.f;
      const float* dB = a.dbuf_out + ((size_t)bh * H + kb) * D * D;
      const float* Sr = a.S_ref + (size_t)bh * D * D;
      for (int i = tid; i < D; i += kThreads) {
        float acc = 0.f, accd = 0.f;
        for (int k = 0; k < D; ++k) { acc += Sr[(size_t)i * D + k] * sphi[k]; accd += dB[(size_t)i * D + k] * sphi[k]; }
        sdel[i] = acc - to_f32(a.v[(tb + pp) * D + i]);
        sdb[i] = accd;
        sdd[i] = cp * accd;
      }
      __syncthreads();
      if (tid == 0 && g.gate_mode == GATE_TOKEN) {
        float du = 0.f;
        for (int i = 0; i < D; ++i) du += sdel[i] * sdb[i];
        for (int j = 0; j < e && pp + j < g.T; ++j) du += p.dw[(tb + pp + j) * e + j];
        a.dgate[tb + pp] = from_f32<T>(du);
      }
      float* dsr = p.dsref_part + ((size_t)bh * sg.nseg + seg) * D * D;
      for (int idx = tid; idx < D * D; idx += kThreads) dsr[idx] += sdd[idx / D] * sphi[idx % D];
    }
    for (int i = tid; i < D; i += kThreads) {
      float val = p.tail_part[tp + i] + (has_next ? p.halo_part[hp + i] : 0.f);
      if (outbuf) val -= sdd[i];
      a.dv[(tb + pp) * D + i] = from_f32<T>(val);
    }
    for (int k = tid; k < D; k += kThreads) {
      float val = p.tail_part[tp + D + k] + (has_next ? p.halo_part[hp + D + k] : 0.f);
      if (outbuf) {
        const float cp = (g.gate_mode == GATE_TOKEN) ? to_f32(a.gate[tb + pp]) : 1.f;
        const float* dB = a.dbuf_out + ((size_t)bh * H + kb) * D * D;
        const float* Sr = a.S_ref + (size_t)bh * D * D;
        float acc = 0.f;
        for (int i = 0; i < D; ++i) acc += cp * dB[(size_t)i * D + k] * sdel[i] + Sr[(size_t)i * D + k] * sdd[i];
        val += acc;
      }
      if (g.map_mode == MAP_ELEMENTWISE) val *= poly_map_grad(to_f32(a.k[(tb + pp) * D + k]), g.map_deg);
      a.dk[(tb + pp) * D + k] = from_f32<T>(val);
    }
  }
  // buffer pass-through when T < e - 1: buffer_out[k'] = buffer_in[T + k']
  if (OUTBUF && seg == 0 && a.dbuf_out && a.dbuf_in && g.T < H) {
    __syncthreads();
    for (int kq = 0; kq + g.T < H; ++kq) {
      const float* src = a.dbuf_out + ((size_t)bh * H + kq) * D * D;
      float* dstb = a.dbuf_in + ((size_t)bh * H + g.T + kq) * D * D;
      for (int idx = tid; idx < D * D; idx += kThreads) dstb[idx] += src[idx];
    }
  }}

}  // namespace atlas
