// mem_params.h - geometry and pointer bundles passed by value to the kernels.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime.h>

namespace atlas {

// Gate modes / map modes mirror atlas_mem.h.
enum { GATE_NONE = 0, GATE_TOKEN = 1, GATE_LAG = 2 };
enum { MAP_OFF = 0, MAP_ELEMENTWISE = 1 };

constexpr int kMaxWindow = 33;  // e <= 33  ->  halo <= 32
constexpr int kHaloPad = 32;    // source tile = chunk + 32 rows

struct Geom {
  int BH, T, DK, DV;
  int e, H;         // window and halo = e - 1
  int Lc;           // chunk length used for this call (<= CH)
  int Lmid;         // forward walk: token offset inside a chunk at which the backward chunks split it
                    // (the backward chunk length when it is Lc / 2), 0 when the chunkings coincide
  int ncb;          // forward walk: number of backward chunks (rows of the saved chunk-start states)
  int nc;           // number of chunks = ceil(T / Lc)
  int momentum, gate_mode, map_mode, map_deg, has_buf, clamp_every, clamp_final;
  // Two launch sequences for one call (scan_chunk_len clamps, see abi.hip): `flag` (device int)
  // selects which one runs. flag_run -1: always run; 0: run only while *flag == 0; 1: only when set.
  // flag_reset: the launch clears *flag first (workgroup 0). clamp_check > 0: set *flag when the
  // unclamped S exceeds 100 in magnitude at a clamp point (every clamp_check tokens, not the last).
  const int* flag;
  int flag_run, flag_reset, clamp_check;
};

// Early exit of a launch whose sequence is not the one the flag selected (a wave-uniform read).
__device__ __forceinline__ bool geom_skip(const Geom& g) {
  if (g.flag_run < 0) return false;
  const int f = *reinterpret_cast<const volatile int*>(g.flag);
  return (f != 0) != (g.flag_run != 0);
}

// The clamp check of the segment-parallel sequence: t1 is a chunk end (the state after token
// t1 - 1); any owned |S| > 100 there means the clamp would change S, so the exact sequence runs.
__device__ __forceinline__ bool clamp_point(const Geom& g, int t1) {
  return g.clamp_check > 0 && t1 < g.T && (t1 % g.clamp_check) == 0;
}
__device__ __forceinline__ void flag_if_clamped(const Geom& g, bool over) {
  if (over) atomicOr(const_cast<int*>(g.flag), 1);
}

// The end of chunk c (token t1 - 1) is a clamp point inside the sequence.
__host__ __device__ inline bool clamp_after(const Geom& g, int t1) {
  return g.clamp_every > 0 && t1 < g.T && (t1 % g.clamp_every) == 0;
}

template <typename T>
struct FwdPtrs {
  const T* k; const T* q; const T* v;
  const T* lr; const T* decay; const T* beta; const T* gate;
  const float* S_ref; const float* S0; const float* Z0; const float* buf_in;
  T* y; float* S_T; float* Z_T; float* buf_out;
  // the specialised walks with a carried buffer: its first-chunk terms (bufwalk.hip), else null
  const float* buf_corr;
};

template <typename T>
struct BwdPtrs {
  const T* k; const T* q; const T* v;
  const T* lr; const T* decay; const T* beta; const T* gate;
  const float* S_ref; const float* S0; const float* Z0; const float* buf_in;
  const T* dy; const float* dS_T; const float* dZ_T; const float* dbuf_out;
  T* dk; T* dq; T* dv; T* dlr; T* ddecay; T* dbeta; T* dgate;
  float* dS_ref; float* dS0; float* dZ0; float* dbuf_in;
};

// Opt-in per-kernel timing (atlas_mem_profile_*): brackets each launch with HIP events.
enum KernelId {
  KID_FWD_SEG_AGG = 0, KID_FWD_WALK, KID_BUFFER_OUT, KID_BWD_ADJOINT, KID_BWD_CHUNK, KID_BWD_FIXUP,
  KID_REDUCE_DSREF, KID_FWD_SCAN, KID_BWD_SCAN, KID_FWD_COEF, KID_BWD_COEF, KID_BWD_SCALAR, KID_BUF_FWD,
  KID_BUF_BWD, KID_COUNT
};
void prof_name(int kid, const char* name);   // records the kernel a stage launches (timing labels)
void prof_begin(int kid, hipStream_t s);
void prof_end(int kid, hipStream_t s);

}  // namespace atlas
