// seg_fwd.hip - segment-parallel forward pass of the chunked memory recurrence (gfx950).
//
// The sequence of every head-batch row bh is cut into segments of G chunks (chunk length Lc).
// Chunk-boundary states follow an affine recurrence with a scalar 2x2 transition,
//   [S; Z]_out = [[a, -kappa], [0, b]] [S; Z]_in + [U; V],
// so the work splits into two launches, both parallel over (segment, bh):
//   k_fwd_seg_agg : walk the segment's chunks from a zero state -> segment aggregate
//                   (a, kappa, b, U_seg, V_seg).
//   k_fwd_seg_scan: one thread per state element (i, k) of a row folds the aggregates in segment
//                   order from (S0, Z0), writing every segment-start state (kept for the backward).
//   k_fwd_seg     : walk the segment's chunks again from its start state, producing y (and S_T,
//                   Z_T in the last segment) and the raw state at every backward-chunk boundary
//                   (kept for the backward pass, which therefore never re-walks the forward).
// With clamp_every > 0 the clamp at scan_chunk_len boundaries is not affine, so the caller uses a
// single segment (an exact sequential walk over all chunks).
//
// Inside a chunk (tokens t0..t1-1, sources s = the chunk plus its e-1 token halo) everything is in
// closed form (the per-chunk coefficients, k_chunk_coef in coef.hip, are formed first):
//   G1  delta^T[s,i] = phi_s . S_ref[i,:] - v_s[i]
//   G2  Q[tau,s]     = Ws[s,tau-1] * (psi_tau . phi_s)
//   G3  y^T[tau,i]   = -Q delta^T + a_{tau-1} psi S_in^T - kappa_{tau-1} psi Z_in^T
//   G4  U = -delta (Ws_end phi), V = delta (Wz_end phi)
//   S_out = a_end S_in - kappa_end Z_in + U,   Z_out = b_end Z_in + V
// Wave roles (8 waves): 0-5 run G1/G2 while 6-7 run the scalar coefficient recurrences; then
// 0-3 run G3 (y) while 4-7 run G4 and keep the 64 x 64 states S, Z in registers.
#include "mem_common.h"
#include "mem_params.h"
#include "seg_common.h"
#include "buffer_out.h"
#include "seg_fwd.h"

namespace atlas {

// Two workgroups per CU (16 waves, at most 128 VGPRs each) for the bf16 configurations, whose
// aggregate-pass LDS fits twice in 160 KB.
template <typename T, int CH, int D>
__global__ __launch_bounds__(kSegThreads) __attribute__((amdgpu_waves_per_eu(4))) void k_fwd_seg_agg(const Geom g, const FwdPtrs<T> a, const SegGeom sg,
                                                               float* agg, const float* coef) {
  if (geom_skip(g)) return;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  fwd_segment<T, CH, D, WALK_AGG>(g, a, sg, agg, nullptr, nullptr, nullptr, coef, nullptr, smem_raw);
}

// grid (D * D / kThreads + H', BH): segment-start states
//   x_{j+1} = [[a_j, -kappa_j], [0, b_j]] x_j + [U_j; V_j],
// and, in the H' = e - 1 workgroups x >= nscan when buffer_out is requested, buffer_out's slot
// x - nscan (buffer_out.h: inputs only, so it rides along with this short launch).
template <typename T, int D>
__global__ __launch_bounds__(kThreads) void k_fwd_seg_scan(const Geom g, const float* S0, const float* Z0,
                                                             const SegGeom sg, const float* agg, float* seg_states,
                                                             const FwdPtrs<T> a, int nscan) {
  if (geom_skip(g)) return;
  const int bh = blockIdx.y;
  if ((int)blockIdx.x >= nscan) {   // workgroup-uniform
    buffer_out_slot<T, D, D>(g, a, blockIdx.x - nscan, bh);
    return;
  }
  const int idx = blockIdx.x * kThreads + threadIdx.x;
  if (idx >= D * D) return;
  float S = S0[(size_t)bh * D * D + idx];
  float Z = (g.momentum && Z0) ? Z0[(size_t)bh * D * D + idx] : 0.f;
  const float* ag = agg + (size_t)bh * sg.nseg * sg.agg_stride;
  float* ss = seg_states + (size_t)bh * sg.nseg * 2 * D * D;
  // aggregates are read kScanBatch segments at a time (one memory round trip per batch)
  for (int j0 = 0; j0 < sg.nseg; j0 += kScanBatch) {
    float U[kScanBatch], V[kScanBatch], ta[kScanBatch], tk[kScanBatch], tbb[kScanBatch];
#pragma unroll
    for (int u = 0; u < kScanBatch; ++u) {
      const float* aj = ag + (size_t)min(j0 + u, sg.nseg - 1) * sg.agg_stride;
      U[u] = aj[idx]; V[u] = aj[D * D + idx];
      ta[u] = aj[2 * D * D]; tk[u] = aj[2 * D * D + 1]; tbb[u] = aj[2 * D * D + 2];
    }
    if (j0 == 0 && a.buf_corr) {   // the specialised walks' carried buffer: its terms at segment 0's end
      const float* bc = a.buf_corr + (size_t)bh * bufw::kCorrFloats;
      U[0] += bc[bufw::AU + idx];
      V[0] += bc[bufw::AV + idx];
    }
#pragma unroll
    for (int u = 0; u < kScanBatch; ++u) {
      const int js = j0 + u;
      if (js < sg.nseg) {
        ss[(size_t)js * 2 * D * D + idx] = S;
        ss[(size_t)js * 2 * D * D + D * D + idx] = Z;
        const float Sn = ta[u] * S - tk[u] * Z + U[u];
        Z = g.momentum ? tbb[u] * Z + V[u] : 0.f;
        S = Sn;
      }
    }
  }
}

template <typename T, int D>
hipError_t launch_fwd_seg_scan(const Geom& g, const FwdPtrs<T>& a, const SegGeom& sg, const float* agg,
                               float* seg_states, hipStream_t stream) {
  const int nscan = (D * D + kThreads - 1) / kThreads;
  const int nbuf = (g.H > 0 && a.buf_out) ? g.H : 0;
  prof_name(KID_FWD_SCAN, nbuf ? "k_fwd_seg_scan+buffer_out" : "k_fwd_seg_scan");
  prof_begin(KID_FWD_SCAN, stream);
  hipLaunchKernelGGL((k_fwd_seg_scan<T, D>), dim3(nscan + nbuf, g.BH), dim3(kThreads), 0, stream, g, a.S0, a.Z0, sg,
                     agg, seg_states, a, nscan);
  prof_end(KID_FWD_SCAN, stream);
  return hipGetLastError();
}
template hipError_t launch_fwd_seg_scan<bf16, 64>(const Geom&, const FwdPtrs<bf16>&, const SegGeom&, const float*,
                                                  float*, hipStream_t);

template <typename T, int CH, int D>
__global__ __launch_bounds__(kSegThreads) void k_fwd_seg(const Geom g, const FwdPtrs<T> a, const SegGeom sg,
                                                           const float* seg_states, float* rw, float* final_raw,
                                                           const float* coef, const T* wsh) {
  if (geom_skip(g)) return;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  fwd_segment<T, CH, D, WALK_FULL>(g, a, sg, nullptr, seg_states, rw, final_raw, coef, wsh, smem_raw);
}

template <typename T, int CH, int D>
hipError_t launch_fwd_seg(const Geom& g, const FwdPtrs<T>& a, const SegGeom& sg, float* agg, float* seg_states,
                          float* rw, float* final_raw, float* coef, T* wsh, hipStream_t stream) {
  // the chunk coefficient records (coef, wsh) are formed by the caller first
  hipError_t err = hipSuccess;
  if (sg.nseg > 1) {
    const size_t smem = sizeof(SegFwdSmem<T, CH, D, false>);
    err = set_dyn_smem(reinterpret_cast<const void*>(&k_fwd_seg_agg<T, CH, D>), smem);
    if (err != hipSuccess) return err;
    prof_name(KID_FWD_SEG_AGG, "k_fwd_seg_agg");
    prof_begin(KID_FWD_SEG_AGG, stream);
    hipLaunchKernelGGL((k_fwd_seg_agg<T, CH, D>), dim3(sg.nseg, g.BH), dim3(kSegThreads), smem, stream, g, a, sg, agg,
                       (const float*)coef);
    prof_end(KID_FWD_SEG_AGG, stream);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  if ((err = launch_fwd_seg_scan<T, D>(g, a, sg, agg, seg_states, stream)) != hipSuccess) return err;
  const size_t smem = sizeof(SegFwdSmem<T, CH, D, true>);
  err = set_dyn_smem(reinterpret_cast<const void*>(&k_fwd_seg<T, CH, D>), smem);
  if (err != hipSuccess) return err;
  prof_name(KID_FWD_WALK, "k_fwd_seg");
  prof_begin(KID_FWD_WALK, stream);
  hipLaunchKernelGGL((k_fwd_seg<T, CH, D>), dim3(sg.nseg, g.BH), dim3(kSegThreads), smem, stream, g, a, sg,
                     (const float*)seg_states, rw, final_raw, (const float*)coef, (const T*)wsh);
  prof_end(KID_FWD_WALK, stream);
  return hipGetLastError();
}

#define ATLAS_INST_FWD_SEG(T, CH, D) \
  template hipError_t launch_fwd_seg<T, CH, D>(const Geom&, const FwdPtrs<T>&, const SegGeom&, float*, float*, float*, \
                                               float*, float*, T*, hipStream_t);

ATLAS_INST_FWD_SEG(bf16, 64, 64)
ATLAS_INST_FWD_SEG(float, 32, 64)
ATLAS_INST_FWD_SEG(bf16, 64, 32)
ATLAS_INST_FWD_SEG(float, 32, 32)

}  // namespace atlas
