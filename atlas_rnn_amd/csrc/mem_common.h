// mem_common.h - device helpers shared by the memory-recurrence kernels (gfx950 / CDNA4).
//
// Matrix-core tiles: every GEMM in this library is an "NT" product
//     C[m, n] = sum_k A[m, k] * Bt[n, k]
// computed as 16x16 output tiles by one wave64 with
//     bf16: v_mfma_f32_16x16x32_bf16 (k step 32, 8 bf16 per lane)
//     fp32: v_mfma_f32_16x16x4_f32   (k step 4, 1 fp32 per lane)
// Lane l of the wave supplies A[m0 + (l & 15)][k0 + (l >> 4) * KL + e] (e < KL) and the same
// pattern of Bt; the accumulator lane l holds C[m0 + 4 * (l >> 4) + i][n0 + (l & 15)], i < 4.
//
// Rule: an MFMA is never issued under a condition whose join is followed by a read of its
// accumulator. With hipcc 7.2 on gfx950 such a join after a conditionally issued
// v_mfma_f32_16x16x4_f32 got too few wait states before v_accvgpr_read, returning the value
// from before the last MFMA. Optional terms are therefore computed unconditionally with zero
// operands (frag_ld_or_zero) instead of being skipped.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <map>
#include <mutex>
#include <utility>

namespace atlas {

// hipFuncSetAttribute(MaxDynamicSharedMemorySize) per kernel and device only when a launch needs
// more than the largest value set so far: the attribute is a maximum, so it is raised and never
// lowered (a launch with fewer bytes after one with more keeps working), and the runtime call does
// not cost host time on every launch.
inline hipError_t set_dyn_smem(const void* fn, size_t bytes) {
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, size_t> raised;
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  const auto key = std::make_pair(fn, dev);
  std::lock_guard<std::mutex> lock(mu);
  const auto it = raised.find(key);
  if (it != raised.end() && it->second >= bytes) return hipSuccess;
  err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (err == hipSuccess) raised[key] = bytes;
  return err;
}


typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

// Workgroup barrier that orders LDS only: waits for this wave's LDS operations (lgkmcnt) but not for
// its global loads, so loads issued ahead (register prefetch) stay in flight across it. For use where
// no other thread reads, after the barrier, global memory this thread wrote before it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

template <typename T> __device__ __forceinline__ float to_f32(T x) { return static_cast<float>(x); }
template <typename T> __device__ __forceinline__ T from_f32(float x) { return static_cast<T>(x); }

template <typename OT> struct MM;

template <> struct MM<bf16> {
  static constexpr int KS = 32;  // k per instruction
  static constexpr int KL = 8;   // k values per lane
  typedef bf16x8 frag;
  static __device__ __forceinline__ f32x4 mma(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <> struct MM<float> {
  static constexpr int KS = 4;
  static constexpr int KL = 1;
  typedef float frag;
  static __device__ __forceinline__ f32x4 mma(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Fragment of a matrix stored with element (r, k) at p[r * rs + k * cs].
template <typename OT, typename ST>
__device__ __forceinline__ typename MM<OT>::frag frag_ld(const ST* p, int rs, int cs, int r0, int k0) {
  const int l = lane_id();
  const ST* q = p + (r0 + (l & 15)) * rs + (k0 + (l >> 4) * MM<OT>::KL) * cs;
  typename MM<OT>::frag f;
  if constexpr (MM<OT>::KL == 1) {
    f = static_cast<OT>(to_f32(q[0]));
  } else {
#pragma unroll
    for (int e = 0; e < MM<OT>::KL; ++e) f[e] = static_cast<OT>(to_f32(q[e * cs]));
  }
  return f;
}

// frag_ld, or a zero fragment when p is null (keeps the MFMA itself unconditional).
template <typename OT, typename ST>
__device__ __forceinline__ typename MM<OT>::frag frag_ld_or_zero(const ST* p, int rs, int cs, int r0, int k0) {
  if (p) return frag_ld<OT>(p, rs, cs, r0, k0);
  typename MM<OT>::frag f;
  if constexpr (MM<OT>::KL == 1) {
    f = static_cast<OT>(0.f);
  } else {
#pragma unroll
    for (int e = 0; e < MM<OT>::KL; ++e) f[e] = static_cast<OT>(0.f);
  }
  return f;
}

// Row-major, k contiguous, same element type: one 16-byte load per lane for bf16.
// Requires rs % 8 == 0 and 16-byte aligned p.
template <typename OT>
__device__ __forceinline__ typename MM<OT>::frag frag_ld_row(const OT* p, int rs, int r0, int k0) {
  const int l = lane_id();
  const OT* q = p + (r0 + (l & 15)) * rs + k0 + (l >> 4) * MM<OT>::KL;
  if constexpr (MM<OT>::KL == 1) {
    return q[0];
  } else {
    return *reinterpret_cast<const typename MM<OT>::frag*>(q);
  }
}

// Same as frag_ld but each k value is multiplied by s[k] (fp32) before rounding to OT.
template <typename OT, typename ST>
__device__ __forceinline__ typename MM<OT>::frag frag_ld_kscaled(const ST* p, int rs, int cs, int r0, int k0,
                                                                const float* s) {
  const int l = lane_id();
  const int kb = k0 + (l >> 4) * MM<OT>::KL;
  const ST* q = p + (r0 + (l & 15)) * rs + kb * cs;
  typename MM<OT>::frag f;
  if constexpr (MM<OT>::KL == 1) {
    f = static_cast<OT>(to_f32(q[0]) * s[kb]);
  } else {
#pragma unroll
    for (int e = 0; e < MM<OT>::KL; ++e) f[e] = static_cast<OT>(to_f32(q[e * cs]) * s[kb + e]);
  }
  return f;
}

// Fragment of a matrix stored transposed in LDS: element (r, k) at p[k * ld + r].
// bf16: two ds_read_b64_tr_b16 (gfx950 transpose loads) per lane instead of eight 2-byte reads.
// Within each 16-lane group g = l >> 4, lane 16g + i supplies the address of the 4 elements
// r0 + 4 (i % 4) .. +3 of row k0 + 8g + h + i / 4 (h = 0, then 4), and lane 16g + m receives
// element m of the group's rows h + j, j < 4: A[r0 + m][k0 + 8g + h + j]. Reads exactly the
// elements frag_ld(p, 1, ld, r0, k0) reads. Requires p in LDS, 8-byte aligned, ld % 4 == 0 and
// r0 % 4 == 0. fp32: the plain strided load (one element per lane).
template <typename OT>
__device__ __forceinline__ typename MM<OT>::frag frag_ld_tr(const OT* p, int ld, int r0, int k0) {
  if constexpr (MM<OT>::KL == 1) {
    return frag_ld<OT>(p, 1, ld, r0, k0);
  } else {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    const int l = lane_id(), i = l & 15;
    const OT* q = p + (k0 + 8 * (l >> 4) + (i >> 2)) * ld + r0 + 4 * (i & 3);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(q));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(q + 4 * ld));
    const s16x8 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(typename MM<OT>::frag, v);
  }
}

// frag_ld_tr with each k value multiplied by s[k] (fp32) before rounding to OT.
template <typename OT>
__device__ __forceinline__ typename MM<OT>::frag frag_ld_tr_kscaled(const OT* p, int ld, int r0, int k0,
                                                                   const float* s) {
  typename MM<OT>::frag f = frag_ld_tr<OT>(p, ld, r0, k0);
  const int kb = k0 + (lane_id() >> 4) * MM<OT>::KL;
  if constexpr (MM<OT>::KL == 1) {
    f = static_cast<OT>(to_f32(f) * s[kb]);
  } else {
#pragma unroll
    for (int e = 0; e < MM<OT>::KL; ++e) f[e] = static_cast<OT>(to_f32(f[e]) * s[kb + e]);
  }
  return f;
}

// Fragment f with its k values scaled by w[k] (w: the KL weights of this lane's k slots).
template <typename T>
__device__ __forceinline__ typename MM<T>::frag frag_scale(typename MM<T>::frag f, const float* w) {
  if constexpr (MM<T>::KL == 1) {
    return f * w[0];
  } else {
    typename MM<T>::frag r;
#pragma unroll
    for (int e = 0; e < MM<T>::KL; ++e) r[e] = static_cast<T>(static_cast<float>(f[e]) * w[e]);
    return r;
  }
}

// Sum over the 16 lanes of each row (lanes 16r .. 16r+15), returned in every lane of the row:
// four DPP row rotations (row_ror 8, 4, 2, 1) on the VALU, no LDS traffic.
__device__ __forceinline__ float row_sum16(float x) {
#define ATLAS_ROR_ADD(n) \
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x120 + (n), 0xf, 0xf, false))
  ATLAS_ROR_ADD(8);
  ATLAS_ROR_ADD(4);
  ATLAS_ROR_ADD(2);
  ATLAS_ROR_ADD(1);
#undef ATLAS_ROR_ADD
  return x;
}

// Eight consecutive values as fp32 (16 bytes of bf16 or 32 of fp32; 16-byte aligned p).
template <typename T>
__device__ __forceinline__ void ld8(const T* p, float* v) {
  if constexpr (sizeof(T) == 2) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const unsigned w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      v[2 * h] = __builtin_bit_cast(float, w[h] << 16);
      v[2 * h + 1] = __builtin_bit_cast(float, w[h] & 0xffff0000u);
    }
  } else {
    const float4 x = reinterpret_cast<const float4*>(p)[0], y = reinterpret_cast<const float4*>(p)[1];
    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w; v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
  }
}
template <typename T>
__device__ __forceinline__ void st8(T* p, const float* v) {
  if constexpr (sizeof(T) == 2) {
    typedef __bf16 bf16x2_ __attribute__((ext_vector_type(2)));
    unsigned w[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      bf16x2_ b;
      b[0] = static_cast<__bf16>(v[2 * h]);
      b[1] = static_cast<__bf16>(v[2 * h + 1]);
      w[h] = __builtin_bit_cast(unsigned, b);
    }
    *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// Clamp of the reference (torch.clamp(-100, 100)) and its gradient mask (min <= x <= max).
__device__ __forceinline__ float clamp100(float x) { return fminf(fmaxf(x, -100.f), 100.f); }
__device__ __forceinline__ float clamp_mask(float x) { return (x >= -100.f && x <= 100.f) ? 1.f : 0.f; }

// Elementwise polynomial feature map sum_{i=1..g} x^i (rnn_memory.py:117-123) and its derivative.
__device__ __forceinline__ float poly_map(float x, int g) {
  float out = x, pw = x;
  for (int i = 2; i <= g; ++i) { pw *= x; out += pw; }
  return out;
}
__device__ __forceinline__ float poly_map_grad(float x, int g) {
  // d/dx sum_{i=1..g} x^i = sum_{i=1..g} i x^{i-1}
  float out = 1.f, pw = 1.f;
  for (int i = 2; i <= g; ++i) { pw *= x; out += static_cast<float>(i) * pw; }
  return out;
}

// Load one element and apply the feature map (identity or elementwise polynomial).
template <typename T>
__device__ __forceinline__ float ld_map(const T* p, size_t idx, int map_mode, int deg) {
  const float x = to_f32(p[idx]);
  return map_mode == 1 ? poly_map(x, deg) : x;
}

}  // namespace atlas
