// fp32 / bf16 MFMA tile helpers for gfx950 (v_mfma_f32_32x32x2f32,
// v_mfma_f32_16x16x4f32, v_mfma_f32_32x32x16_bf16) shared by the chunk kernels.
//
// Operand feeding.  A 32x32x2 MFMA step takes one A and one B value per lane:
// A(row l%32, c), B(c, col l%32) with c = 2 s + l/32.  mma8 instead feeds,
// over four steps s = 0..3, contraction index c0 + s with c0 = 8 g + 4 (l/32):
// the same 8 indices of group g, permuted.  A lane then needs four consecutive
// contraction values of one row or column: one vector LDS read when the
// contraction axis is contiguous (ld_c), four conflict-free scalar reads when
// the row axis is (ld_x).  The accumulator of a 32x32 tile holds, in lane l
// register r, row 8 (r/4) + 4 (l/32) + r%4 and column l%32 (acc_row); the
// bf16 32x32x16 MFMA uses the same accumulator layout with lane l holding row
// (or column) l%32 and contraction indices 8 (l/32) .. +7 of each 16-step.
#pragma once
#include <hip/hip_runtime.h>

#include "gdn_common.h"

namespace gpa {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));


__device__ __forceinline__ void mma8(f32x16& c, f32x4 a, f32x4 b) {
  c = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b.x, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b.y, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b.z, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b.w, c, 0, 0, 0);
}

// 16x16x4 with the same permutation: lane quarter q = l/16 feeds c0 + s, c0 = 16 g + 4 q.
__device__ __forceinline__ void mma16(f32x4& c, f32x4 a, f32x4 b) {
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, c, 0, 0, 0);
}

// Element (x, c0 + s), s = 0..3, of a matrix stored with c contiguous ...
__device__ __forceinline__ f32x4 ld_c(const float* m, int ld, int x, int c0) {
  return *reinterpret_cast<const f32x4*>(m + x * ld + c0);
}
// ... or with x contiguous.
__device__ __forceinline__ f32x4 ld_x(const float* m, int ld, int x, int c0) {
  return f32x4{m[c0 * ld + x], m[(c0 + 1) * ld + x], m[(c0 + 2) * ld + x], m[(c0 + 3) * ld + x]};
}

__device__ __forceinline__ int acc_row(int r, int half) { return 8 * (r >> 2) + 4 * half + (r & 3); }

// Sums of each of a lane's 16 accumulator-row values over the 32 lanes of its
// half-wave, by recursive halving (16 exchanges instead of 16 x 5).  Every
// lane returns the sum for register index sum_index(lane).
__device__ __forceinline__ float tile_row_sum(float (&v)[16], int lane) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const bool up = lane & 16;
    const float send = up ? v[j] : v[j + 8], keep = up ? v[j + 8] : v[j];
    v[j] = keep + __shfl_xor(send, 16);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool up = lane & 8;
    const float send = up ? v[j] : v[j + 4], keep = up ? v[j + 4] : v[j];
    v[j] = keep + __shfl_xor(send, 8);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const bool up = lane & 4;
    const float send = up ? v[j] : v[j + 2], keep = up ? v[j + 2] : v[j];
    v[j] = keep + __shfl_xor(send, 4);
  }
  {
    const bool up = lane & 2;
    const float send = up ? v[0] : v[1], keep = up ? v[1] : v[0];
    v[0] = keep + __shfl_xor(send, 2);
  }
  return v[0] + __shfl_xor(v[0], 1);
}
__device__ __forceinline__ int sum_index(int lane) {
  return 8 * ((lane >> 4) & 1) + 4 * ((lane >> 3) & 1) + 2 * ((lane >> 2) & 1) + ((lane >> 1) & 1);
}

// Four consecutive activation-type elements as floats (8 bytes for bf16).
__device__ __forceinline__ f32x4 ld_c(const bf16_t* m, int ld, int x, int c0) {
  const uint2 w = *reinterpret_cast<const uint2*>(m + x * ld + c0);
  return f32x4{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u), __uint_as_float(w.y << 16),
               __uint_as_float(w.y & 0xffff0000u)};
}

template <typename E>
__device__ __forceinline__ E op_raw(const gpa_operand& o, int b, int h, int t, int d) {
  return reinterpret_cast<const E*>(o.ptr)[op_base(o, b, h) + (int64_t)t * o.st + d];
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Eight consecutive floats rounded to bf16 (round to nearest even).
__device__ __forceinline__ bf16x8 pack8(const float* x) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(x), c = *reinterpret_cast<const f32x4*>(x + 4);
  bf16x8 r;
  r[0] = (__bf16)a.x; r[1] = (__bf16)a.y; r[2] = (__bf16)a.z; r[3] = (__bf16)a.w;
  r[4] = (__bf16)c.x; r[5] = (__bf16)c.y; r[6] = (__bf16)c.z; r[7] = (__bf16)c.w;
  return r;
}

// Split bf16 operands of v_mfma_f32_32x32x16_bf16 (lane l: row or column
// l%32, contraction 8 (l/32) .. +7).  An fp32 value x is carried as hi + lo,
// hi = bf16(x), lo = bf16(x - hi); a product keeps hi*hi + hi*lo + lo*hi,
// about 16 significant bits.  Values exact in bf16 go in unsplit.
struct SplitBf8 {
  bf16x8 hi, lo;
};
// Eight floats as bf16 hi and lo vectors (element e of x is element e of each).
__device__ __forceinline__ void split8(const float (&x)[8], bf16x8& hi, bf16x8& lo) {
  uint32_t h[4], o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) bf2_split(x[2 * i], x[2 * i + 1], h[i], o[i]);
  __builtin_memcpy(&hi, h, 16);
  __builtin_memcpy(&lo, o, 16);
}
__device__ __forceinline__ SplitBf8 split_bf8(const float (&x)[8]) {
  SplitBf8 s;
  split8(x, s.hi, s.lo);
  return s;
}
// Elements (c0 + e, x), e = 0..7, of an fp32 matrix stored with x contiguous.
__device__ __forceinline__ SplitBf8 col_split_bf8(const float* m, int ld, int x, int c0) {
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = m[(c0 + e) * ld + x];
  return split_bf8(v);
}
// Elements (x, c0 + e) of an fp32 matrix stored with c contiguous (16-byte aligned rows).
__device__ __forceinline__ SplitBf8 row_split_bf8(const float* m, int ld, int x, int c0) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(m + x * ld + c0), b = *reinterpret_cast<const f32x4*>(m + x * ld + c0 + 4);
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  return split_bf8(v);
}
// Elements (x, c0 + e) of a bf16 matrix stored with c contiguous (8-byte aligned rows).
__device__ __forceinline__ bf16x8 row_bf8(const bf16_t* m, int ld, int x, int c0) {
  const uint2 a = *reinterpret_cast<const uint2*>(m + x * ld + c0), b = *reinterpret_cast<const uint2*>(m + x * ld + c0 + 4);
  const uint4 w = make_uint4(a.x, a.y, b.x, b.y);
  bf16x8 r;
  __builtin_memcpy(&r, &w, 16);
  return r;
}
__device__ __forceinline__ void mma_bf16(f32x16& c, bf16x8 a, bf16x8 b) {
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ void mma_split(f32x16& c, const SplitBf8& a, const SplitBf8& b) {
  mma_bf16(c, a.hi, b.hi);
  mma_bf16(c, a.hi, b.lo);
  mma_bf16(c, a.lo, b.hi);
}
__device__ __forceinline__ void mma_exact_split(f32x16& c, bf16x8 a, const SplitBf8& b) {
  mma_bf16(c, a, b.hi);
  mma_bf16(c, a, b.lo);
}
__device__ __forceinline__ void mma_split_exact(f32x16& c, const SplitBf8& a, bf16x8 b) {
  mma_bf16(c, a.hi, b);
  mma_bf16(c, a.lo, b);
}

template <typename E>
__device__ __forceinline__ f32x4 round4(f32x4 x) {
  return f32x4{round_as<E>(x.x), round_as<E>(x.y), round_as<E>(x.z), round_as<E>(x.w)};
}

}  // namespace gpa
