// Host build of a HIP kernel source (test infrastructure, never shipped).
//
// Each workgroup runs as blockDim.x std::threads that share the kernel's
// __shared__ objects (made static: one workgroup runs at a time);
// __syncthreads is a barrier over them, and a wave shuffle exchanges through a
// per-wave buffer between two barriers of that wave's 64 threads.  Built with
// AddressSanitizer, every global access of the kernel is checked against the
// exact extent of the buffer it addresses.
#pragma once
#include <hip/hip_runtime_api.h>

#include <atomic>
#include <barrier>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <memory>
#include <thread>
#include <tuple>
#include <vector>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __shared__ static
#define __launch_bounds__(...)
#define __align__(n) __attribute__((aligned(n)))

struct dim3 {
  unsigned x = 1, y = 1, z = 1;
  dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
struct uint2 {
  unsigned x, y;
};
struct uint4 {
  unsigned x, y, z, w;
};
inline uint4 make_uint4(unsigned a, unsigned b, unsigned c, unsigned d) { return uint4{a, b, c, d}; }
struct float4 {
  float x, y, z, w;
};
inline float4 make_float4(float a, float b, float c, float d) { return float4{a, b, c, d}; }
struct EmuIdx {
  unsigned x, y, z;
};
extern thread_local EmuIdx threadIdx, blockIdx, blockDim, gridDim;
extern std::barrier<>* emu_block_barrier;
extern std::vector<std::unique_ptr<std::barrier<>>> emu_wave_barrier;
extern float emu_xchg[16][64];

inline void __syncthreads() { emu_block_barrier->arrive_and_wait(); }
inline float __shfl_xor(float v, int m, int width = 64) {
  (void)width;  // m < width keeps the partner inside the segment
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  emu_xchg[w][l] = v;
  emu_wave_barrier[w]->arrive_and_wait();
  const float r = emu_xchg[w][l ^ m];
  emu_wave_barrier[w]->arrive_and_wait();
  return r;
}
// __shfl_up / __shfl_down / __shfl: lanes whose source falls outside their
// width-lane segment keep their own value (up, down); __shfl reads lane
// `src` of the segment.
inline float emu_shfl_from(float v, int src) {
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  emu_xchg[w][l] = v;
  emu_wave_barrier[w]->arrive_and_wait();
  const float r = emu_xchg[w][src];
  emu_wave_barrier[w]->arrive_and_wait();
  return r;
}
inline float __shfl_up(float v, unsigned d, int width = 64) {
  const int l = threadIdx.x % 64;
  return emu_shfl_from(v, (l % width) >= (int)d ? l - (int)d : l);
}
inline float __shfl_down(float v, unsigned d, int width = 64) {
  const int l = threadIdx.x % 64;
  return emu_shfl_from(v, (l % width) + (int)d < width ? l + (int)d : l);
}
inline float __shfl(float v, int src, int width = 64) {
  const int l = threadIdx.x % 64;
  return emu_shfl_from(v, l - l % width + src % width);
}
inline float atomicAdd(float* p, float v) { return std::atomic_ref<float>(*p).fetch_add(v); }

// MFMA: every lane posts its operands, then computes its own accumulator
// registers from the whole wave's operands (lane layouts of the gfx950
// instructions: A(row l%32, k), B(k, col l%32), accumulator lane l register r
// at row 8(r/4) + 4(l/32) + r%4, column l%32; 16x16x4: A(row l%16, k = l/16),
// accumulator row 4(l/16) + r).
typedef float emu_f32x4 __attribute__((ext_vector_type(4)));
typedef float emu_f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 emu_bf16x8 __attribute__((ext_vector_type(8)));
extern float emu_ma[16][64][8], emu_mb[16][64][8];
inline void emu_post(const float* a, const float* b, int n) {
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  for (int i = 0; i < n; ++i) {
    emu_ma[w][l][i] = a[i];
    emu_mb[w][l][i] = b[i];
  }
  emu_wave_barrier[w]->arrive_and_wait();
}
inline emu_f32x16 emu_mfma_32x32x16_bf16(emu_bf16x8 a, emu_bf16x8 b, emu_f32x16 c) {
  float fa[8], fb[8];
  for (int i = 0; i < 8; ++i) {
    fa[i] = (float)a[i];
    fb[i] = (float)b[i];
  }
  emu_post(fa, fb, 8);
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  for (int r = 0; r < 16; ++r) {
    const int row = 8 * (r / 4) + 4 * (l / 32) + r % 4, col = l % 32;
    float s = 0.f;
    for (int k = 0; k < 16; ++k) s += emu_ma[w][row + 32 * (k / 8)][k % 8] * emu_mb[w][col + 32 * (k / 8)][k % 8];
    c[r] += s;
  }
  emu_wave_barrier[w]->arrive_and_wait();
  return c;
}
inline emu_f32x16 emu_mfma_32x32x2_f32(float a, float b, emu_f32x16 c) {
  emu_post(&a, &b, 1);
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  for (int r = 0; r < 16; ++r) {
    const int row = 8 * (r / 4) + 4 * (l / 32) + r % 4, col = l % 32;
    c[r] += emu_ma[w][row][0] * emu_mb[w][col][0] + emu_ma[w][row + 32][0] * emu_mb[w][col + 32][0];
  }
  emu_wave_barrier[w]->arrive_and_wait();
  return c;
}
inline emu_f32x4 emu_mfma_16x16x4_f32(float a, float b, emu_f32x4 c) {
  emu_post(&a, &b, 1);
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  for (int r = 0; r < 4; ++r) {
    const int row = 4 * (l / 16) + r, col = l % 16;
    float s = 0.f;
    for (int k = 0; k < 4; ++k) s += emu_ma[w][row + 16 * k][0] * emu_mb[w][col + 16 * k][0];
    c[r] += s;
  }
  emu_wave_barrier[w]->arrive_and_wait();
  return c;
}
#define __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, x, y, z) emu_mfma_32x32x16_bf16(a, b, c)
// Only used on values that are uniform over the wave, where it is the identity.
#define __builtin_amdgcn_readfirstlane(x) (x)
// v_perm_b32: byte i of the result is byte sel.byte[i] of {a (bytes 4-7), b
// (bytes 0-3)}, or 0x00 for selector 0x0c (the only other selector used).
inline uint32_t emu_perm(uint32_t a, uint32_t b, uint32_t sel) {
  const uint64_t c = ((uint64_t)a << 32) | b;
  uint32_t d = 0;
  for (int i = 0; i < 4; ++i) {
    const uint32_t s = (sel >> (8 * i)) & 0xff;
    if (s != 0x0c && s > 7) abort();
    const uint32_t byte = s == 0x0c ? 0u : (uint32_t)((c >> (8 * s)) & 0xff);
    d |= byte << (8 * i);
  }
  return d;
}
#define __builtin_amdgcn_perm(a, b, s) emu_perm((uint32_t)(a), (uint32_t)(b), (uint32_t)(s))
#define __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, x, y, z) emu_mfma_32x32x2_f32(a, b, c)
#define __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, x, y, z) emu_mfma_16x16x4_f32(a, b, c)

// Dynamic LDS: an allocation of exactly the launch's size per workgroup.
extern char* emu_dynamic_lds;
#define HIP_DYNAMIC_SHARED(type, var) type* var = reinterpret_cast<type*>(emu_dynamic_lds);
#define hipSuccess 0
#define hipFuncAttributeMaxDynamicSharedMemorySize 8
inline int hipFuncSetAttribute(const void*, int, int) { return 0; }

// The runtime calls of the scan library's host code.  Launches run to
// completion here, one after another, so streams and events order nothing:
// they are opaque non-null handles.  The device is one MI355X (256 CUs).
typedef int hipDevice_t;
enum hipStreamCaptureStatus { hipStreamCaptureStatusNone = 0, hipStreamCaptureStatusActive = 1 };
#define hipStreamNonBlocking 1u
#define hipEventDisableTiming 2u
#define hipDeviceAttributeMultiprocessorCount 63
inline hipError_t hipGetDevice(int* d) {
  *d = 0;
  return hipSuccess;
}
inline hipError_t hipSetDevice(int) { return hipSuccess; }
inline hipError_t hipDeviceGetAttribute(int* v, int, int) {
  *v = 256;
  return hipSuccess;
}
inline hipError_t hipStreamGetDevice(hipStream_t, hipDevice_t* d) {
  *d = 0;
  return hipSuccess;
}
inline hipError_t hipStreamIsCapturing(hipStream_t, hipStreamCaptureStatus* s) {
  *s = hipStreamCaptureStatusNone;
  return hipSuccess;
}
inline char emu_handles[2];
inline hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned) {
  *s = reinterpret_cast<hipStream_t>(&emu_handles[0]);
  return hipSuccess;
}
inline hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned) {
  *e = reinterpret_cast<hipEvent_t>(&emu_handles[1]);
  return hipSuccess;
}
inline hipError_t hipEventRecord(hipEvent_t, hipStream_t) { return hipSuccess; }
inline hipError_t hipStreamWaitEvent(hipStream_t, hipEvent_t, unsigned) { return hipSuccess; }
inline const char* hipGetErrorString(hipError_t) { return "host build"; }
#define HIP_SYMBOL(x) (&(x))
inline hipError_t hipGetSymbolAddress(void** p, const void* symbol) {
  *p = const_cast<void*>(symbol);
  return hipSuccess;
}
inline float __expf(float x) { return expf(x); }
// correctly rounded single operations (the host build is compiled without FMA contraction)
inline float __fadd_rn(float a, float b) { return a + b; }
inline float __fsub_rn(float a, float b) { return a - b; }
inline float __fmul_rn(float a, float b) { return a * b; }
inline float __fdiv_rn(float a, float b) { return a / b; }
inline float __uint_as_float(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
inline uint32_t __float_as_uint(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

// Inline assembly: the kernels' only statement is `asm volatile("s_waitcnt
// lgkmcnt(0)\n\ts_barrier" ::: "memory")` (the LDS-only barrier).  Here
// `asm` vanishes and `volatile(...)` becomes a call that sees the statement's
// text: a barrier over the workgroup when it holds s_barrier, else nothing (a
// wait for outstanding memory operations is implicit on the host).
inline void emu_asm(const char* text) {
  if (strstr(text, "s_barrier")) __syncthreads();
}
#define asm
#define volatile(...) emu_asm(#__VA_ARGS__)

// The kernel-argument segment: the address of the running kernel's first
// argument (each emulated thread holds its own copy of the arguments).
extern thread_local const void* emu_kernarg;
#define __builtin_amdgcn_kernarg_segment_ptr() (emu_kernarg)

template <typename K, typename... A>
void emu_launch(K kernel, dim3 grid, dim3 block, size_t lds_bytes, A... args) {
  // One team of blockDim.x threads runs the workgroups one after another; a
  // barrier separates workgroups (their __shared__ objects are shared statics).
  const unsigned nt = block.x;
  std::barrier<> bar(nt), between(nt);
  emu_block_barrier = &bar;
  emu_wave_barrier.clear();
  for (unsigned w = 0; w < (nt + 63) / 64; ++w) emu_wave_barrier.emplace_back(new std::barrier<>(64));
  std::vector<char> lds(lds_bytes ? lds_bytes : 1);
  emu_dynamic_lds = lds.data();
  std::vector<std::thread> threads;
  for (unsigned t = 0; t < nt; ++t)
    threads.emplace_back([&, t] {
      const std::tuple<A...> targs(args...);
      emu_kernarg = &std::get<0>(targs);
      threadIdx = {t, 0, 0};
      blockDim = {block.x, block.y, block.z};
      gridDim = {grid.x, grid.y, grid.z};
      for (unsigned bz = 0; bz < grid.z; ++bz)
        for (unsigned by = 0; by < grid.y; ++by)
          for (unsigned bx = 0; bx < grid.x; ++bx) {
            blockIdx = {bx, by, bz};
            std::apply(kernel, targs);
            between.arrive_and_wait();
          }
    });
  for (auto& th : threads) th.join();
}
#define hipLaunchKernelGGL(k, g, b, s, st, ...) emu_launch(k, g, b, s, __VA_ARGS__)
