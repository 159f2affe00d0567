// Shared device helpers and host error reporting for libgpa_hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gpa {

// bfloat16 is carried as its bit pattern.
struct bf16_t {
  uint16_t bits;
};

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return __uint_as_float((uint32_t)x.bits << 16); }

// Round-to-nearest-even float -> bfloat16 (a NaN stays a NaN): the hardware
// conversion (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  const __bf16 h = (__bf16)f;
  bf16_t r;
  __builtin_memcpy(&r, &h, sizeof r);
  return r;
}

template <typename E> __device__ __forceinline__ E from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) { return f32_to_bf16(x); }

// One IEEE operation, rounded on its own: the compiler may not fuse these into
// an FMA (the pragma strips the contraction flag from the operation), which the
// reference's separately rounded products and sums require.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ __forceinline__ float sub_rn(float a, float b) {
#pragma clang fp contract(off)
  return a - b;
}
__device__ __forceinline__ float div_rn(float a, float b) {
#pragma clang fp contract(off)
  return a / b;
}

// Value after a round trip through E: the reference rounds normalised keys and
// queries to the activation dtype before the fp32 state arithmetic.
template <typename E> __device__ __forceinline__ float round_as(float x) { return to_f32(from_f32<E>(x)); }

}  // namespace gpa

// Host side: thread-local last error and launch checking (defined in abi.hip).
int fail(int code, const char* message);
int check_launch(const char* what);

// Records timing->events[timing->launched++] on `stream` (no-op without timing).
struct gpa_timing;
void mark(gpa_timing* timing, hipStream_t stream);

namespace gpa {
// Up to four products C[h] = sum over the R rows r of A[h][r]^T B[h][r]
// (float32 [heads][a_width][b_width], cleared first), rounded to bf16 values
// when bf16: row r of head h of A sits at a + h * a_hs + r * a_rs (elements).
// The bf16 path runs them as one MFMA launch (route_reader.hip).
struct TnProduct {
  const void* a;
  int64_t a_rs, a_hs;
  int a_width;
  const void* b;
  int64_t b_rs, b_hs;
  int b_width;
  float* c;
};
int launch_tn_products(const TnProduct* products, int n, int heads, int rows, bool bf16, hipStream_t stream);
}  // namespace gpa
