// chunk_fwd.hip - forward pass of the chunk-parallel path (chunk_common.h): three launches.
//
//   k_cp_agg   (segment, row): the segment's zero-start end state (U, V) and its transition, as one
//              product over all of the segment's sources (no walk over its chunks)
//   k_cp_scan  (element, row): segment-start states from the aggregates; S_T / Z_T / the raw
//              S_{T-1}; buffer_out in extra workgroups
//   k_cp_out   (chunk, row): the chunk-start state (segment-start state carried over the segment's
//              earlier chunks: one product over their sources), then y for the chunk's 64 tokens
//
// Per chunk (targets t = 0 .. 63 at tokens t0 + t, sources s = -16 .. 63 at tokens t0 + s):
//   y_t = At S_c psi_t + Kt Z_c psi_t + sum_s Wy[s][t] (phi_s . psi_t) delta_s
//   delta_s = S_ref phi_s - v_s,   At, Kt: coefficients of S_c, Z_c in S_{t-1}
//   Wy[s][t] = sum_j w(s + j, j) C'[s + j][t]: coefficient of G_s = delta_s phi_s^T in S_{t-1}
//   C'[r][t] = -sum_{u = r .. t-1} B(r -> u) eta_u A(u -> t-1): coefficient of g_r in S_{t-1}
// C' and Wy are matrix products whose operands are formed in registers from the chunk's log2
// prefix sums (exp2 of differences) and its gates, so no coefficient table is stored anywhere.
#include "chunk_common.h"
#include "buffer_out.h"

namespace atlas {

namespace cp {

// Own-chunk shared memory of k_cp_out (gates follow it, dynamically sized).
struct OutSm {
  alignas(16) bf16 phi[SRC][PD];    // sources t0 - 16 .. t0 + 63 (mapped)
  alignas(16) bf16 psi[CL][PD];     // targets (mapped)
  alignas(16) bf16 vd[SRC][PD];     // v of the sources, then delta in place
  alignas(16) bf16 blk[2][CL][PD];  // staging of the earlier chunks' phi / v; then S_c^T, Z_c^T ([k][i])
  RangeSm rs;
  float la[CL], lb[CL], eta[CL];    // chunk-local log2 prefix sums of alpha / beta; eta
  float At[CL], Kt[CL];
};

struct AggSm {
  alignas(16) bf16 blk[2][CL][PD];
  RangeSm rs;
};

// gate floats staged for a range of n targets (lag) or its n + HT sources (token)
__host__ __device__ inline int gate_floats(int gate_mode, int e, int n) {
  return gate_mode == GATE_LAG ? n * e : (gate_mode == GATE_TOKEN ? n + HT : 0);
}

}  // namespace cp

using namespace cp;

// ---------------------------------------------------------------------------------------------
// k_cp_agg: grid (nseg, BH)
// ---------------------------------------------------------------------------------------------
template <bool MAPE>
__global__ __launch_bounds__(NTH) void k_cp_agg(const Geom g, const FwdPtrs<bf16> a, const SegGeom sg, float* agg) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  AggSm& sm = *reinterpret_cast<AggSm*>(smem_raw);
  float* gates = reinterpret_cast<float*>(smem_raw + carry_offset<AggSm>());
  const int seg = blockIdx.x, bh = blockIdx.y, w = wave_id();
  const int ta = seg * SEGT, n = min(SEGT, g.T - ta);
  const size_t rowbase = (size_t)bh * g.T;
  const uint32_t row_bytes = (uint32_t)g.T * (D * 2);
  const rsrc_t rk = make_rsrc(a.k + rowbase * D, row_bytes);
  const rsrc_t rv = make_rsrc(a.v + rowbase * D, row_bytes);
  // every global load of the workgroup first: sources, scalars, S_ref, gates
  SrcBlocks<5> sb;
  src_load<5>(sb, rk, rv, ta - HT, n + HT);
  const TokScal sc = range_scalars(g, a.decay, a.lr, a.beta, rowbase, ta, n);
  bf16x8 sref[2];
  load_sref(a.S_ref + (size_t)bh * D * D, w, sref);
  stage_gates(g, a.gate, rowbase, ta, n, gates, gates);
  __syncthreads();
  range_coefs(g, sc, ta, n, sm.rs, gates, gates);
  __syncthreads();
  f32x4 Sacc[4], Zacc[4];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) { Sacc[kt] = zero4(); Zacc[kt] = zero4(); }
  state_blocks<MAPE, 5>(sb, n + HT, sm.rs, sref, &sm.blk[0][0][0], &sm.blk[1][0][0], Sacc, Zacc, g.map_deg);
  const int lane = lane_id(), gq = lane >> 4, m = lane & 15;
  float* ag = agg + ((size_t)bh * sg.nseg + seg) * sg.agg_stride;
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int off = (16 * w + 4 * gq + r) * D + 16 * kt + m;
      ag[off] = Sacc[kt][r];
      ag[D * D + off] = g.momentum ? Zacc[kt][r] : 0.f;
    }
  if (threadIdx.x == 0) {
    const Tri tr = sm.rs.trans;
    ag[2 * D * D] = tr.a;
    ag[2 * D * D + 1] = -tr.k;   // S_out = a S_in - kappa Z_in + U
    ag[2 * D * D + 2] = tr.b;
  }
}

// ---------------------------------------------------------------------------------------------
// k_cp_scan: grid (D * D / 256 + H', BH). Segment-start states, then the final state.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_cp_scan(const Geom g, const FwdPtrs<bf16> a, const SegGeom sg,
                                                  const float* agg, float* seg_states, float* final_raw, int nscan) {
  const int bh = blockIdx.y;
  if ((int)blockIdx.x >= nscan) {   // workgroup-uniform
    buffer_out_slot<bf16, D, D>(g, a, blockIdx.x - nscan, bh);
    return;
  }
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= D * D) return;
  const size_t sb = (size_t)bh * D * D + idx;
  float S = a.S0[sb];
  float Z = (g.momentum && a.Z0) ? a.Z0[sb] : 0.f;
  const float* ag = agg + (size_t)bh * sg.nseg * sg.agg_stride;
  float* ss = seg_states + (size_t)bh * sg.nseg * 2 * D * D;
  for (int j0 = 0; j0 < sg.nseg; j0 += kScanBatch) {
    float U[kScanBatch], V[kScanBatch], ta[kScanBatch], tk[kScanBatch], tb[kScanBatch];
#pragma unroll
    for (int u = 0; u < kScanBatch; ++u) {
      const float* aj = ag + (size_t)min(j0 + u, sg.nseg - 1) * sg.agg_stride;
      U[u] = aj[idx]; V[u] = aj[D * D + idx];
      ta[u] = aj[2 * D * D]; tk[u] = aj[2 * D * D + 1]; tb[u] = aj[2 * D * D + 2];
    }
#pragma unroll
    for (int u = 0; u < kScanBatch; ++u) {
      const int js = j0 + u;
      if (js < sg.nseg) {
        ss[(size_t)js * 2 * D * D + idx] = S;
        ss[(size_t)js * 2 * D * D + D * D + idx] = Z;
        const float Sn = ta[u] * S - tk[u] * Z + U[u];
        Z = g.momentum ? tb[u] * Z + V[u] : 0.f;
        S = Sn;
      }
    }
  }
  a.S_T[sb] = g.clamp_final ? clamp100(S) : S;
  if (g.momentum && a.Z_T) a.Z_T[sb] = Z;
  if (final_raw) final_raw[sb] = S;
}

// ---------------------------------------------------------------------------------------------
// k_cp_out: grid (nc, BH)
// ---------------------------------------------------------------------------------------------
template <bool MAPE, bool MOM>
__global__ __launch_bounds__(NTH) void k_cp_out(const Geom g, const FwdPtrs<bf16> a, const SegGeom sg,
                                                 const float* seg_states) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  OutSm& sm = *reinterpret_cast<OutSm*>(smem_raw);
  float* gates = reinterpret_cast<float*>(smem_raw + carry_offset<OutSm>());
  const int c = blockIdx.x, bh = blockIdx.y;
  const int tid = threadIdx.x, lane = lane_id(), w = wave_id(), gq = lane >> 4, m = lane & 15;
  const int t0 = c * CL, seg = c / SEGC, st0 = seg * SEGT;
  const int nr = t0 - st0;                  // earlier targets of the segment
  const size_t rowbase = (size_t)bh * g.T;
  const uint32_t row_bytes = (uint32_t)g.T * (D * 2);
  const rsrc_t rk = make_rsrc(a.k + rowbase * D, row_bytes);
  const rsrc_t rq = make_rsrc(a.q + rowbase * D, row_bytes);
  const rsrc_t rv = make_rsrc(a.v + rowbase * D, row_bytes);
  const rsrc_t ry = make_rsrc(a.y + rowbase * D, row_bytes);

  // ---- own chunk in flight: phi and v rows t0 - 16 .. t0 + 63, psi rows t0 .. t0 + 63
  // (vector index v: tensor rows v / 8, column chunk v % 8; 7 vectors per thread)
  constexpr int NV_SRC = SRC * 8, NV_PSI = CL * 8;   // 640, 512
  constexpr int NV = 2 * NV_SRC + NV_PSI;            // 1792
  constexpr int PER = NV / NTH;                      // 7
  static_assert(NV % NTH == 0, "vectors per thread");
  u32x4v own[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int v = tid + u * NTH;
    if (v < NV_SRC) {
      own[u] = bld16(rk, (uint32_t)((t0 - HT + v / 8) * (D * 2) + (v % 8) * 16));
    } else if (v < 2 * NV_SRC) {
      const int x = v - NV_SRC;
      own[u] = bld16(rv, (uint32_t)((t0 - HT + x / 8) * (D * 2) + (x % 8) * 16));
    } else {
      const int x = v - 2 * NV_SRC;
      own[u] = bld16(rq, (uint32_t)((t0 + x / 8) * (D * 2) + (x % 8) * 16));
    }
  }
  bf16x8 sref[2];
  load_sref(a.S_ref + (size_t)bh * D * D, w, sref);
  // the earlier chunks' sources, the range scalars, the segment-start state (all in flight at once)
  SrcBlocks<SEGC> sb;
  src_load<SEGC>(sb, rk, rv, st0 - HT, nr > 0 ? nr + HT : 0);
  const TokScal rsc = range_scalars(g, a.decay, a.lr, a.beta, rowbase, st0, nr);
  float s0v[4][4], z0v[4][4];
  {
    const float* ss = seg_states + ((size_t)bh * sg.nseg + seg) * 2 * D * D;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int off = (16 * w + 4 * gq + r) * D + 16 * kt + m;
        s0v[kt][r] = ss[off];
        z0v[kt][r] = MOM ? ss[D * D + off] : 0.f;
      }
  }

  // ---- gates of targets st0 .. t0 + 63 (and their sources); chunk scalars
  stage_gates(g, a.gate, rowbase, st0, nr + CL, gates, gates);
  if (w == 0) {
    const TokScal sc = tok_scalars(g, a.decay, a.lr, a.beta, rowbase, t0 + lane);
    const float la = wave_prefix_sum(fmaxf(__log2f(sc.al), kLogFloor), lane);
    sm.la[lane] = la;
    sm.eta[lane] = sc.et;
    if (MOM) sm.lb[lane] = wave_prefix_sum(fmaxf(__log2f(sc.be), kLogFloor), lane);
    // (At, Kt): first row of M_{t-1} ... M_0
    const Tri inc = wave_scan<true>(Tri{sc.al, -sc.et * sc.be, sc.be}, lane);
    Tri ex = tri_prev_lane(inc);
    if (lane == 0) ex = tri_id();
    sm.At[lane] = ex.a;
    sm.Kt[lane] = ex.k;
  }
  __syncthreads();
  if (nr > 0) {
    range_coefs(g, rsc, st0, nr, sm.rs, gates, gates);
  } else if (tid == 0) {
    sm.rs.trans = tri_id();
  }
  // ---- own chunk to LDS
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int v = tid + u * NTH;
    if (v < NV_SRC) {
      u32x4v x = own[u];
      if constexpr (MAPE) x = map_bf16x8(x, g.map_deg);
      *reinterpret_cast<u32x4v*>(&sm.phi[v / 8][(v % 8) * 8]) = x;
    } else if (v < 2 * NV_SRC) {
      const int x = v - NV_SRC;
      *reinterpret_cast<u32x4v*>(&sm.vd[x / 8][(x % 8) * 8]) = own[u];
    } else {
      const int x = v - 2 * NV_SRC;
      u32x4v y = own[u];
      if constexpr (MAPE) y = map_bf16x8(y, g.map_deg);
      *reinterpret_cast<u32x4v*>(&sm.psi[x / 8][(x % 8) * 8]) = y;
    }
  }
  __syncthreads();

  // ---- chunk-start state: the segment-start state carried over the earlier chunks of the segment
  f32x4 Sacc[4], Zacc[4];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) { Sacc[kt] = zero4(); Zacc[kt] = zero4(); }
  state_blocks<MAPE, SEGC>(sb, nr > 0 ? nr + HT : 0, sm.rs, sref, &sm.blk[0][0][0], &sm.blk[1][0][0], Sacc, Zacc,
                           g.map_deg);
  {
    const Tri tr = sm.rs.trans;
    float Sv[4][4], Zv[4][4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        Sv[kt][r] = tr.a * s0v[kt][r] + tr.k * z0v[kt][r] + Sacc[kt][r];
        Zv[kt][r] = MOM ? tr.b * z0v[kt][r] + Zacc[kt][r] : 0.f;
      }
    __syncthreads();   // every wave is done with the staging buffers
    bf16* ScT = &sm.blk[0][0][0];
    bf16* ZcT = &sm.blk[1][0][0];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      store4<bf16>(ScT + (16 * kt + m) * PD + 16 * w + 4 * gq, Sv[kt][0], Sv[kt][1], Sv[kt][2], Sv[kt][3]);
      store4<bf16>(ZcT + (16 * kt + m) * PD + 16 * w + 4 * gq, Zv[kt][0], Zv[kt][1], Zv[kt][2], Zv[kt][3]);
    }
  }

  // ---- delta of the chunk's sources (rows i of this wave), in place of v
#pragma unroll
  for (int st = 0; st < SRC / 16; ++st) {
    f32x4 acc = zero4();
#pragma unroll
    for (int q = 0; q < 2; ++q) acc = mma_bf16(sref[q], frag_row(&sm.phi[0][0], PD, 16 * st, 32 * q), acc);
    bf16* p = &sm.vd[16 * st + m][16 * w + 4 * gq];
    const float4 vv = lds_bf16x4(p);
    store4<bf16>(p, acc[0] - vv.x, acc[1] - vv.y, acc[2] - vv.z, acc[3] - vv.w);
  }

  // ---- this wave's 16 targets t = 16 w + m: C', Wy, K^T, Q
  const int tt = w;
  f32x4 cpr[4];
  const bf16x8 fdec[2] = {gen_decay_to(sm.la, 16 * tt + m, 0, lane), gen_decay_to(sm.la, 16 * tt + m, 1, lane)};
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
    cpr[rt] = zero4();
#pragma unroll
    for (int q = 0; q < 2; ++q) cpr[rt] = mma_bf16(gen_beta_eta<MOM>(sm.lb, sm.eta, 16 * rt + m, q, lane), fdec[q], cpr[rt]);
  }
  const float* wl_own = gates + (size_t)nr * g.e;   // lag gates of targets t0 ..
  const float* ug_own = gates + nr;                 // token gates of sources t0 - 16 ..
  bf16x8 fq[3];
  {
    const bf16x8 fc0 = pack_frag(cpr[0], cpr[1]), fc1 = pack_frag(cpr[2], cpr[3]);
    f32x4 Q[SRC / 16];
#pragma unroll
    for (int st = 0; st < SRC / 16; ++st) {
      f32x4 wy = zero4(), kq = zero4();
      wy = mma_bf16(gen_wgate(g, wl_own, ug_own, t0, 16 * st + m, 0, lane), fc0, wy);
      wy = mma_bf16(gen_wgate(g, wl_own, ug_own, t0, 16 * st + m, 1, lane), fc1, wy);
#pragma unroll
      for (int q = 0; q < 2; ++q)
        kq = mma_bf16(frag_row(&sm.phi[0][0], PD, 16 * st, 32 * q), frag_row(&sm.psi[0][0], PD, 16 * tt, 32 * q), kq);
#pragma unroll
      for (int r = 0; r < 4; ++r) Q[st][r] = kq[r] * wy[r];
    }
    fq[0] = pack_frag(Q[0], Q[1]);
    fq[1] = pack_frag(Q[2], Q[3]);
    fq[2] = pack_frag(Q[4], zero4());
  }
  __syncthreads();   // delta and S_c^T / Z_c^T of every wave

  // ---- y^T[i][t] for the wave's targets, all rows i
  const bf16* ScT = &sm.blk[0][0][0];
  const bf16* ZcT = &sm.blk[1][0][0];
  const int t = 16 * tt + m;
  const float At = sm.At[t], Kt = sm.Kt[t];
  bf16x8 fpsi[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) fpsi[q] = frag_row(&sm.psi[0][0], PD, 16 * tt, 32 * q);
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    f32x4 yi = zero4(), ys = zero4(), yz = zero4();
    yi = mma_bf16(tr_pair<true>(&sm.vd[0][0], PD, 0, 16 * it), fq[0], yi);
    yi = mma_bf16(tr_pair<true>(&sm.vd[0][0], PD, 1, 16 * it), fq[1], yi);
    yi = mma_bf16(tr_pair<false>(&sm.vd[0][0], PD, 2, 16 * it), fq[2], yi);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      ys = mma_bf16(frag_ld_tr<bf16>(ScT, PD, 16 * it, 32 * q), fpsi[q], ys);
      yz = mma_bf16(frag_ld_tr<bf16>(ZcT, PD, 16 * it, 32 * q), fpsi[q], yz);
    }
    u32x2v out;
    out[0] = pack_bf16x2(yi[0] + At * ys[0] + Kt * yz[0], yi[1] + At * ys[1] + Kt * yz[1]);
    out[1] = pack_bf16x2(yi[2] + At * ys[2] + Kt * yz[2], yi[3] + At * ys[3] + Kt * yz[3]);
    bst8(ry, (uint32_t)(((t0 + t) * D + 16 * it + 4 * gq) * 2), out);
  }
}

// ---------------------------------------------------------------------------------------------

bool chunk_path_supported(const Geom& g) {
  return g.DK == D && g.DV == D && g.H <= HT && g.clamp_every == 0 && g.clamp_check == 0 && !g.has_buf &&
         g.flag_run < 0;
}

SegGeom chunk_seg(const Geom& g) {
  SegGeom s{};
  s.G = SEGC;
  s.nseg = (g.nc + SEGC - 1) / SEGC;
  s.agg_stride = 2 * D * D + 16;
  return s;
}

template <bool MAPE, bool MOM>
static hipError_t launch_out(const Geom& g, const FwdPtrs<bf16>& a, const SegGeom& sg, const float* seg_states,
                             hipStream_t stream) {
  const size_t smem = carry_offset<OutSm>() + sizeof(float) * gate_floats(g.gate_mode, g.e, SEGT);
  hipError_t err = set_dyn_smem(reinterpret_cast<const void*>(&k_cp_out<MAPE, MOM>), smem);
  if (err != hipSuccess) return err;
  prof_name(KID_FWD_WALK, "k_cp_out");
  prof_begin(KID_FWD_WALK, stream);
  hipLaunchKernelGGL((k_cp_out<MAPE, MOM>), dim3(g.nc, g.BH), dim3(NTH), smem, stream, g, a, sg, seg_states);
  prof_end(KID_FWD_WALK, stream);
  return hipGetLastError();
}

// The forward of the chunk-parallel path. The gates, the aggregates and the segment-start states
// are laid out by sg = chunk_seg(g); final_raw receives the unclamped S_{T-1}.
hipError_t launch_chunk_fwd(const Geom& g, const FwdPtrs<bf16>& a, const SegGeom& sg, float* agg, float* seg_states,
                            float* final_raw, hipStream_t stream) {
  const bool mape = g.map_mode == MAP_ELEMENTWISE;
  hipError_t err;
  {
    const size_t smem = carry_offset<AggSm>() + sizeof(float) * gate_floats(g.gate_mode, g.e, SEGT);
    const void* fn = mape ? reinterpret_cast<const void*>(&k_cp_agg<true>) : reinterpret_cast<const void*>(&k_cp_agg<false>);
    if ((err = set_dyn_smem(fn, smem)) != hipSuccess) return err;
    prof_name(KID_FWD_SEG_AGG, "k_cp_agg");
    prof_begin(KID_FWD_SEG_AGG, stream);
    if (mape) hipLaunchKernelGGL((k_cp_agg<true>), dim3(sg.nseg, g.BH), dim3(NTH), smem, stream, g, a, sg, agg);
    else hipLaunchKernelGGL((k_cp_agg<false>), dim3(sg.nseg, g.BH), dim3(NTH), smem, stream, g, a, sg, agg);
    prof_end(KID_FWD_SEG_AGG, stream);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  {
    const int nscan = (D * D + 255) / 256;
    const int nbuf = (g.H > 0 && a.buf_out) ? g.H : 0;
    prof_name(KID_FWD_SCAN, nbuf ? "k_cp_scan+buffer_out" : "k_cp_scan");
    prof_begin(KID_FWD_SCAN, stream);
    hipLaunchKernelGGL(k_cp_scan, dim3(nscan + nbuf, g.BH), dim3(256), 0, stream, g, a, sg, (const float*)agg,
                       seg_states, final_raw, nscan);
    prof_end(KID_FWD_SCAN, stream);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  if (mape) return g.momentum ? launch_out<true, true>(g, a, sg, seg_states, stream)
                              : launch_out<true, false>(g, a, sg, seg_states, stream);
  return g.momentum ? launch_out<false, true>(g, a, sg, seg_states, stream)
                    : launch_out<false, false>(g, a, sg, seg_states, stream);
}

}  // namespace atlas
