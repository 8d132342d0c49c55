// walk_common.h - helpers of the specialised (bf16, d = 64) segment walks.
//
// Raw buffer accesses: every per-row tensor is addressed through a buffer resource whose
// num_records is the row's byte size, so a load outside the row (a negative offset before the
// first token, a token at or past T) returns zeros and a store outside it is dropped by the
// hardware range check. The walks therefore load halo and tail rows unconditionally, with no
// masks, selects or clamped addresses.
//
// Chained matrix-core operands: the A and B fragments of v_mfma_f32_16x16x32_bf16 share one lane
// layout (lane l supplies row l & 15, eight k slots (l >> 4) * 8 + e), and a 16 x 16 accumulator
// holds C[4 (l >> 4) + r][l & 15]. Two vertically adjacent accumulator tiles (rows 32q .. 32q+15
// and 32q+16 .. 32q+31) therefore form one operand fragment over k = 32q .. 32q+31 when the k slots
// are taken in the order
//   slot (g, e):  k = 32q + 4g + e        (e < 4, from the upper tile)
//                 k = 32q + 16 + 4g + e-4 (e >= 4, from the lower tile)
// A sum over k does not depend on the order of its terms, so the partner operand only has to be
// loaded in the same order (tr_pair below). Products such as (S_ref phi^T) -> delta -> delta W phi
// thus pass from one MFMA to the next in registers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mem_common.h"

namespace atlas {

typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef unsigned u32x4v __attribute__((__vector_size__(16)));
typedef unsigned u32x2v __attribute__((__vector_size__(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kOob = 0x80000000u;   // voffset that is always out of range (loads read zero)

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  // word 3 = 0x00020000: raw (untyped) 32-bit data format, as required for buffer_load_dword*
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ u32x4v bld16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}
__device__ __forceinline__ u32x2v bld8(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
}
__device__ __forceinline__ unsigned short bld2(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}
__device__ __forceinline__ void bst8(rsrc_t r, uint32_t off, u32x2v v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, (int)off, 0, 0);
}
__device__ __forceinline__ void bst16(rsrc_t r, uint32_t off, u32x4v v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)off, 0, 0);
}

__device__ __forceinline__ float bf16_bits_to_f32(unsigned short h) {
  return __builtin_bit_cast(float, (unsigned)h << 16);
}

// Two fp32 values rounded to bf16 and packed (low half = a).
__device__ __forceinline__ unsigned pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 v;
  v[0] = static_cast<__bf16>(a);
  v[1] = static_cast<__bf16>(b);
  return __builtin_bit_cast(unsigned, v);
}

// Operand fragment from two accumulator tiles (see the slot order above), each value scaled.
__device__ __forceinline__ bf16x8 pack_frag(const f32x4& hi, const f32x4& lo) {
  bf16x8 f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    f[r] = static_cast<__bf16>(hi[r]);
    f[4 + r] = static_cast<__bf16>(lo[r]);
  }
  return f;
}
__device__ __forceinline__ bf16x8 pack_frag_scaled(const f32x4& hi, const f32x4& lo, const float4& shi,
                                                   const float4& slo) {
  bf16x8 f;
  f[0] = static_cast<__bf16>(hi[0] * shi.x); f[1] = static_cast<__bf16>(hi[1] * shi.y);
  f[2] = static_cast<__bf16>(hi[2] * shi.z); f[3] = static_cast<__bf16>(hi[3] * shi.w);
  f[4] = static_cast<__bf16>(lo[0] * slo.x); f[5] = static_cast<__bf16>(lo[1] * slo.y);
  f[6] = static_cast<__bf16>(lo[2] * slo.z); f[7] = static_cast<__bf16>(lo[3] * slo.w);
  return f;
}
__device__ __forceinline__ bf16x8 zero_frag() {
  bf16x8 f;
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = static_cast<__bf16>(0.f);
  return f;
}

// gfx950 transposing LDS read (ds_read_b64_tr_b16) of a row-major bf16 matrix p[row][col] (pitch
// ld elements): lane (g = l >> 4, m = l & 15) receives p[row0 + 4g + j][col0 + m], j < 4.
// Address lane (g, i) points at the 4 elements col0 + 4 (i & 3) .. +3 of row row0 + 4g + (i >> 2).
// Requires p in LDS, 8-byte aligned rows (ld % 4 == 0) and col0 % 4 == 0.
__device__ __forceinline__ s16x4 tr4(const bf16* p, int ld, int row0, int col0) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const int l = lane_id(), g = l >> 4, i = l & 15;
  const bf16* q = p + (row0 + 4 * g + (i >> 2)) * ld + col0 + 4 * (i & 3);
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(q));
}

// Operand fragment over k = 32q .. 32q+31 in the chained slot order, read transposed from a
// row-major p[k][col]: lane (g, m) gets p[32q + 4g + j][col0 + m] (slots j) and
// p[32q + 16 + 4g + j][col0 + m] (slots 4 + j). LO = false leaves the lower half zero (rows past
// the end of p).
template <bool LO = true>
__device__ __forceinline__ bf16x8 tr_pair(const bf16* p, int ld, int q, int col0) {
  const s16x4 a = tr4(p, ld, 32 * q, col0);
  s16x4 b = s16x4{0, 0, 0, 0};
  if constexpr (LO) b = tr4(p, ld, 32 * q + 16, col0);
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const s16x8 v = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, v);
}

// Four bf16 values at p (8-byte aligned, LDS) as fp32.
__device__ __forceinline__ float4 lds_bf16x4(const bf16* p) {
  const uint2 u = *reinterpret_cast<const uint2*>(p);
  return make_float4(__builtin_bit_cast(float, u.x << 16), __builtin_bit_cast(float, u.x & 0xffff0000u),
                     __builtin_bit_cast(float, u.y << 16), __builtin_bit_cast(float, u.y & 0xffff0000u));
}

__device__ __forceinline__ f32x4 mma_bf16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Row-major fragment (16-byte LDS read): lane supplies p[r0 + (l & 15)][k0 + 8 (l >> 4) .. +7].
__device__ __forceinline__ bf16x8 frag_row(const bf16* p, int ld, int r0, int k0) {
  const int l = lane_id();
  return *reinterpret_cast<const bf16x8*>(p + (r0 + (l & 15)) * ld + k0 + 8 * (l >> 4));
}

// The same fragment reads with the lane index passed in. Inside a chunk loop the caller passes a
// lane index laundered through an empty asm statement once per chunk, so that the per-lane LDS
// addresses are recomputed each chunk instead of being hoisted out of the loop and held in (or
// spilled from) registers for the whole walk.
__device__ __forceinline__ int launder(int x) {
  asm volatile("" : "+v"(x));
  return x;
}
__device__ __forceinline__ float launder_f(float x) {
  asm volatile("" : "+v"(x));
  return x;
}
__device__ __forceinline__ bf16x8 frag_row_l(const bf16* p, int ld, int r0, int k0, int l) {
  return *reinterpret_cast<const bf16x8*>(p + (r0 + (l & 15)) * ld + k0 + 8 * (l >> 4));
}
// lane (g, m) receives p[row0 + 4g + j][col0 + m], j < 4 (see tr4)
__device__ __forceinline__ s16x4 tr4_l(const bf16* p, int ld, int row0, int col0, int l) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const int g = l >> 4, i = l & 15;
  const bf16* q = p + (row0 + 4 * g + (i >> 2)) * ld + col0 + 4 * (i & 3);
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(q));
}
// Standard-order fragment of the transpose of a row-major p[k][r]: lane supplies
// A[r0 + (l & 15)][k0 + 8 (l >> 4) + e] = p[k0 + 8 (l >> 4) + e][r0 + (l & 15)] (two transposing reads).
__device__ __forceinline__ bf16x8 frag_tr_l(const bf16* p, int ld, int r0, int k0, int l) {
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  // tr4_l adds 4 (l >> 4) to the row base: rows k0 + 8 (l >> 4) + (0..3), then + 4 .. 7
  const s16x4 lo = tr4_l(p, ld, k0 + 4 * (l >> 4), r0, l);
  const s16x4 hi = tr4_l(p, ld, k0 + 4 * (l >> 4) + 4, r0, l);
  const s16x8 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, v);
}
// frag_tr_l with k value e scaled by s[k0 + 8 (l >> 4) + e] (fp32, LDS).
__device__ __forceinline__ bf16x8 frag_tr_scaled_l(const bf16* p, int ld, int r0, int k0, const float* s, int l) {
  const bf16x8 f = frag_tr_l(p, ld, r0, k0, l);
  const float4 s0 = *reinterpret_cast<const float4*>(s + k0 + 8 * (l >> 4));
  const float4 s1 = *reinterpret_cast<const float4*>(s + k0 + 8 * (l >> 4) + 4);
  bf16x8 r;
  r[0] = static_cast<__bf16>(static_cast<float>(f[0]) * s0.x); r[1] = static_cast<__bf16>(static_cast<float>(f[1]) * s0.y);
  r[2] = static_cast<__bf16>(static_cast<float>(f[2]) * s0.z); r[3] = static_cast<__bf16>(static_cast<float>(f[3]) * s0.w);
  r[4] = static_cast<__bf16>(static_cast<float>(f[4]) * s1.x); r[5] = static_cast<__bf16>(static_cast<float>(f[5]) * s1.y);
  r[6] = static_cast<__bf16>(static_cast<float>(f[6]) * s1.z); r[7] = static_cast<__bf16>(static_cast<float>(f[7]) * s1.w);
  return r;
}

template <bool LO = true>
__device__ __forceinline__ bf16x8 tr_pair_l(const bf16* p, int ld, int q, int col0, int l) {
  const s16x4 a = tr4_l(p, ld, 32 * q, col0, l);
  s16x4 b = s16x4{0, 0, 0, 0};
  if constexpr (LO) b = tr4_l(p, ld, 32 * q + 16, col0, l);
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const s16x8 v = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, v);
}

// Sum of x over the four 16-lane rows of the wave (lanes m, m + 16, m + 32, m + 48), returned in
// every lane: two gfx950 cross-row swaps (v_permlane32_swap, v_permlane16_swap) on the VALU
// instead of LDS-routed lane shuffles. Written as inline assembly because the compiler's
// two-result builtins were seen to drop the second result when both operands hold the same value;
// the leading s_nop covers the VALU-write -> permlane-read hazard.
__device__ __forceinline__ float xsum_rows(float x) {
  float a = x, b = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  float c = a + b, d = c;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(c), "+v"(d));
  return c + d;
}

// Elementwise polynomial map on eight bf16 values held as a 16-byte vector.
__device__ __forceinline__ u32x4v map_bf16x8(u32x4v v, int deg) {
  u32x4v r;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float a = poly_map(__builtin_bit_cast(float, v[w] << 16), deg);
    const float b = poly_map(__builtin_bit_cast(float, v[w] & 0xffff0000u), deg);
    r[w] = pack_bf16x2(a, b);
  }
  return r;
}

// Saved chunk-start states of the specialised walks (forward -> backward): per backward chunk,
// S then Z, each 64 x 64 bf16 stored as eight 1 KB operand fragments (kt = 0..3, q = 0..1) in the
// chained slot order: lane (g, m) of fragment (kt, q) holds X[32q + 4g + r][16kt + m] in slots r < 4
// and X[32q + 16 + 4g + r][16kt + m] in slots 4 + r. The backward loads a fragment with one 16-byte
// access per lane; the forward's state owners (16-row tile it, columns 16kt + m) write 8 bytes.
constexpr int kStateBytes = 64 * 64 * 2;        // one state, bf16
constexpr int kStateBlk = 2 * kStateBytes;      // S and Z of one backward chunk
__device__ __forceinline__ uint32_t frag_off(int kt, int q, int lane) {
  return (uint32_t)(((kt * 2 + q) * 64 + lane) * 16);
}

}  // namespace atlas
