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
#include <vector>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __shared__ static
#define __launch_bounds__(...)

struct dim3 {
  unsigned x = 1, y = 1, z = 1;
  dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
struct EmuIdx {
  unsigned x, y, z;
};
extern thread_local EmuIdx threadIdx, blockIdx;
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
inline float atomicAdd(float* p, float v) { return std::atomic_ref<float>(*p).fetch_add(v); }
inline float __expf(float x) { return expf(x); }
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

template <typename K, typename... A>
void emu_launch(K kernel, dim3 grid, dim3 block, A... args) {
  const unsigned nt = block.x;
  for (unsigned bx = 0; bx < grid.x; ++bx) {
    std::barrier<> bar(nt);
    emu_block_barrier = &bar;
    emu_wave_barrier.clear();
    for (unsigned w = 0; w < (nt + 63) / 64; ++w) emu_wave_barrier.emplace_back(new std::barrier<>(64));
    std::vector<std::thread> threads;
    for (unsigned t = 0; t < nt; ++t)
      threads.emplace_back([=] {
        threadIdx = {t, 0, 0};
        blockIdx = {bx, 0, 0};
        kernel(args...);
      });
    for (auto& th : threads) th.join();
  }
}
#define hipLaunchKernelGGL(k, g, b, s, st, ...) emu_launch(k, g, b, __VA_ARGS__)
