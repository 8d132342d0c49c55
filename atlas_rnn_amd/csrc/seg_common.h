// seg_common.h - pieces shared by the segment-parallel kernels.
#pragma once

#include "mem_common.h"
#include "mem_params.h"

namespace atlas {

constexpr int kSegThreads = 512;   // 8 waves per workgroup
constexpr int kSegWaves = kSegThreads / kWave;
constexpr int kScanBatch = 8;   // segment aggregates loaded per round trip by the segment scans

struct SegGeom {
  int G;              // chunks per segment
  int nseg;           // segments per head-batch row
  int agg_stride;     // floats per segment aggregate: U, V (2 D^2) + a, kappa, b (padded to 16)
};

// The adjoint aggregates of the specialised backward are formed over the forward's 64-token
// chunks (an aggregate does not depend on how its segment is chunked, so this halves the serial
// steps), with the forward's coefficient records: the forward geometry, segments and records.
// chunk_bwd: the reverse walk is k_cp_bwd (chunk_bwd.hip) over the forward's chunks and segments,
// with its coefficients formed in the kernel (no backward records, saved boundary states or
// scalar-gradient inputs), followed by its own fixup.
struct AggOverFwd {
  Geom g;
  SegGeom sg;
  const float* coef;
  bool chunk_bwd;
};

// Backward-pass buffers beyond the user-visible arguments.
struct BwdSegPtrs {
  const float* seg_states;   // forward segment-start states [BH][nseg][2][D][D]
  const float* final_raw;    // forward raw S_{T-1} [BH][D][D]
  float* adj_agg;            // [BH][nseg][agg_stride]: L, K, a, kappa, b
  float* seg_adj;            // [BH][nseg][2][D][D] adjoint (dS, dZ) at each segment end
  const float* rw;           // [BH][nc][2][D][D] raw chunk-start states (written by the forward walk)
  float* dsref_part;         // [BH][nseg][D][D]
  float* tail_part;          // [BH][nseg][H][2D]  (dv | dphi) partial of a segment's last H tokens
  float* halo_part;          // [BH][nseg][H][2D]  partial from the segment's first chunk for the previous segment
  float* dw;                 // [BH][T][e] per (target, lag) gradients (token gates)
  float* coef;               // [BH][nc][CoefRec] chunk coefficient records (k_chunk_coef)
  void* wsh;                 // [BH][nc][CH][SPM] Ws[s, t-1] of every chunk (input element type)
  float* scal;               // [BH][nc][ScalarBlock] per-chunk inputs of the scalar gradients
  float* buf_adj;            // [BH][2][D][D] first chunk's end adjoint (specialised walk with a carried buffer)
};

// The carried buffer on the specialised walks (bufwalk.hip, d = 64). Per row, its first-chunk terms:
// the state corrections after the forward chunk's last token (end) and after token Lmid - 1 (mid),
// and the same end terms carried to the end of segment 0 (added to its aggregate by the segment scan).
namespace bufw {
constexpr int D = 64, CHF = 64, CHB = 32;
constexpr int SE = 0, ZE = D * D, SM = 2 * D * D, ZM = 3 * D * D, AU = 4 * D * D, AV = 5 * D * D;
constexpr int kCorrFloats = 6 * D * D;
constexpr int kAdjFloats = 2 * D * D;
}

// Per backward chunk, written by the reverse walk and read by k_bwd_scalar (fp32):
//   Lm[q][s] = (dy_q . delta_s)(psi_q . phi_s)   [CH][SPM]
//   hS[s] = <dS_end, delta_s phi_s^T>, hZ[s] = <dZ_end, delta_s phi_s^T>   (dense buffer sources: <., B_s>)
//   fS[q] = psi_q . (S_in^T dy_q), fZ[q] = psi_q . (Z_in^T dy_q)
//   gram = <dS_end, S_in>, <dS_end, Z_in>, <dZ_end, Z_in>
template <int CH>
struct ScalarBlock {
  static constexpr int SPM = CH + kHaloPad;
  static constexpr int LM = 0, HS = CH * SPM, HZ = HS + SPM, FS = HZ + SPM, FZ = FS + CH, GRAM = FZ + CH;
  static constexpr int SIZE = GRAM + 4;
  static_assert(SIZE % 4 == 0, "16-byte aligned blocks");
};

// Window weight of the source t - j for target t: the token gate of the source, the lag gate
// w[t][j], or 1.
__device__ __forceinline__ float src_w(int gate_mode, float ug, const float* wl, int e, int t, int j) {
  return gate_mode == GATE_TOKEN ? ug : (gate_mode == GATE_LAG ? wl[t * e + j] : 1.f);
}

// Eight consecutive elements: one 16-byte (bf16) or two 16-byte (fp32) vector accesses.
template <typename T>
struct Vec8 {
  T v[8];
  static __device__ __forceinline__ Vec8 zero() {
    Vec8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r.v[e] = static_cast<T>(0.f);
    return r;
  }
  __device__ __forceinline__ Vec8 mapped(int deg) const {
    Vec8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r.v[e] = static_cast<T>(poly_map(to_f32(v[e]), deg));
    return r;
  }
  // every element times w, rounded to T, stored to 16-byte aligned p (built as words, so no
  // aggregate temporary goes through scratch)
  __device__ __forceinline__ void store_scaled(T* p, float w) const {
    if constexpr (sizeof(T) == 2) {
      unsigned wd[4];
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const unsigned lo = __builtin_bit_cast(unsigned short, static_cast<T>(to_f32(v[2 * h]) * w));
        const unsigned hi = __builtin_bit_cast(unsigned short, static_cast<T>(to_f32(v[2 * h + 1]) * w));
        wd[h] = lo | (hi << 16);
      }
      *reinterpret_cast<uint4*>(p) = make_uint4(wd[0], wd[1], wd[2], wd[3]);
    } else {
      reinterpret_cast<float4*>(p)[0] = make_float4(to_f32(v[0]) * w, to_f32(v[1]) * w, to_f32(v[2]) * w, to_f32(v[3]) * w);
      reinterpret_cast<float4*>(p)[1] = make_float4(to_f32(v[4]) * w, to_f32(v[5]) * w, to_f32(v[6]) * w, to_f32(v[7]) * w);
    }
  }
  // this vector if ok, zeros otherwise (word-wise selects, no aggregate temporaries)
  __device__ __forceinline__ Vec8 masked(bool ok) const {
    Vec8 r;
    constexpr int NW = sizeof(v) / 4;
    const unsigned* src = reinterpret_cast<const unsigned*>(v);
    unsigned* dst = reinterpret_cast<unsigned*>(r.v);
#pragma unroll
    for (int w = 0; w < NW; ++w) dst[w] = ok ? src[w] : 0u;
    return r;
  }
  __device__ __forceinline__ void store(T* p) const {
    if constexpr (sizeof(T) == 2) {
      *reinterpret_cast<uint4*>(p) = *reinterpret_cast<const uint4*>(v);
    } else {
      reinterpret_cast<uint4*>(p)[0] = reinterpret_cast<const uint4*>(v)[0];
      reinterpret_cast<uint4*>(p)[1] = reinterpret_cast<const uint4*>(v)[1];
    }
  }
};

// Four values rounded to T and stored contiguously (8 bytes for bf16, 16 for fp32; p aligned).
template <typename T>
__device__ __forceinline__ void store4(T* p, float a, float b, float c, float d) {
  if constexpr (sizeof(T) == 2) {
    typedef T t4 __attribute__((ext_vector_type(4)));
    t4 v;
    v[0] = static_cast<T>(a); v[1] = static_cast<T>(b); v[2] = static_cast<T>(c); v[3] = static_cast<T>(d);
    *reinterpret_cast<t4*>(p) = v;
  } else {
    *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
  }
}

// Eight fp32 values to / from 16-byte aligned memory (two 16-byte accesses).
__device__ __forceinline__ void store8f(float* p, const float* v) {
  reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
  reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
}
__device__ __forceinline__ void add8f(float* v, const float* p) {
  const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
  v[0] += a.x; v[1] += a.y; v[2] += a.z; v[3] += a.w;
  v[4] += b.x; v[5] += b.y; v[6] += b.z; v[7] += b.w;
}

// Byte offset of dynamic data placed after a shared-memory struct, rounded up to 16 bytes.
template <typename Sm>
constexpr size_t carry_offset() { return (sizeof(Sm) + 15) & ~(size_t)15; }

template <typename T>
__device__ __forceinline__ Vec8<T> vec8_load(const T* p) {
  Vec8<T> r;
  if constexpr (sizeof(T) == 2) {
    *reinterpret_cast<uint4*>(r.v) = *reinterpret_cast<const uint4*>(p);
  } else {
    reinterpret_cast<uint4*>(r.v)[0] = reinterpret_cast<const uint4*>(p)[0];
    reinterpret_cast<uint4*>(r.v)[1] = reinterpret_cast<const uint4*>(p)[1];
  }
  return r;
}

// Per-chunk scalars and coefficients in LDS.
template <int CH>
struct ChunkScalars {
  static constexpr int SPM = CH + kHaloPad;
  float alpha[CH], eta[CH], beta[CH];   // padded targets: alpha = beta = 1, eta = 0
  float ug[SPM];                        // token-mode gate of each source
  float wl[CH * kMaxWindow];            // lag-mode weights [tau][j]
  // the coefficient record (same order as CoefRec, one contiguous 16-byte aligned block)
  alignas(16) float acoef[CH];          // a_{tau-1}
  float kcoef[CH];                      // kappa_{tau-1}
  float endc[4];                        // a_end, kappa_end, b_end
  float wsend[SPM], wzend[SPM];         // Ws[s, end], Wz[s, end]
  float wsmid[SPM], wzmid[SPM];         // Ws[s, Lmid-1], Wz[s, Lmid-1] (zero when Lmid == 0)
  float midc[4];                        // a, kappa, b after token Lmid-1
};

// Per-chunk coefficient record in HBM (fp32), written by k_chunk_coef for every chunk of every row:
// acoef[CH], kcoef[CH], endc[4], wsend[SPM], wzend[SPM], wsmid[SPM], wzmid[SPM], midc[4] - the
// layout of ChunkScalars from acoef on.
template <int CH>
struct CoefRec {
  static constexpr int SPM = CH + kHaloPad;
  static constexpr int SIZE = 2 * CH + 8 + 4 * SPM;   // floats
  static_assert(SIZE % 4 == 0, "record copied as float4");
};

// Decay tables of one chunk, stored [c][t] with source column c = t' + 1 (column 0 is the chunk
// start, t' = -1) and target row t:
//   A[c][t] = prod_{u = t'+1 .. t} alpha_u,   B[c][t] = prod_{u = t'+1 .. t} beta_u,
//   C[c][t] = response of Ws at t to a unit input into Wz at t':
//             C[c][t'] = eta_t',  C[c][t] = alpha_t C[c][t-1] + eta_t B[c][t]   (t > t'),
// and zero for t < t'. Column 0 holds the chunk-start coefficients a_t, b_t, kappa_t. Every linear
// recurrence along the chunk (Wz / Ws of a source, and the adjoint recurrences of the scalar
// gradients) is a sum over these columns, so it runs in parallel instead of step by step.
// The pitch CH + 1 keeps row-wise and column-wise accesses free of bank conflicts.
template <int CH>
struct DecayTab {
  float A[CH + 1][CH + 1], B[CH + 1][CH + 1], C[CH + 1][CH + 1];
};

// Lane t's value of x, in every lane (v_readlane; t is a wave-uniform constant).
__device__ __forceinline__ float lane_bcast(float x, int t) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), t));
}

// Decay tables of a chunk, computed by one wave with one column per lane (lane c = 0..CH;
// lanes above CH run the same chain and write nothing). Column c (tp = c - 1), for t >= tp:
//   A[c][t] = prod_{r=c..t} alpha_r,  B[c][t] = prod_{r=c..t} beta_r,
//   C[c][t] = alpha_t C[c][t-1] + eta_t B[c][t]   (C[c][tp] = eta_tp),
// zero for t < tp. Lane 0 also writes B1[t] = b_{t-1} (t = 0..CH, B1[0] = 1). The step scalars
// are read once into lane t's registers and broadcast with v_readlane, so the chains never wait
// on LDS reads (the table writes are not waited on).
template <int CH>
__device__ __forceinline__ void decay_columns_wave(DecayTab<CH>& tab, const ChunkScalars<CH>& sc, float* B1) {
  static_assert(CH < kWave, "one lane per column");
  const int c = lane_id(), tp = c - 1;
  const bool writer = c <= CH;
  const int ts = c < CH ? c : 0;
  const float al_v = sc.alpha[ts], et_v = sc.eta[ts], be_v = sc.beta[ts];
  float a = 1.f, b = 1.f, m = 0.f;
  if (c == 0) B1[0] = 1.f;
#pragma unroll
  for (int t = 0; t < CH; ++t) {
    const float al = lane_bcast(al_v, t), et = lane_bcast(et_v, t), be = lane_bcast(be_v, t);
    if (t == tp) {
      m = et;
    } else if (t > tp) {
      b = be * b;
      a = al * a;
      m = al * m + et * b;
    }
    const bool on = t >= tp;
    if (writer) {
      tab.A[c][t] = on ? a : 0.f;
      tab.B[c][t] = on ? b : 0.f;
      tab.C[c][t] = on ? m : 0.f;
    }
    if (c == 0) B1[t + 1] = b;
  }
}

}  // namespace atlas
