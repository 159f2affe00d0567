// Elementwise sum of up to GPA_SUM_MAX equally sized buffers, accumulated in
// float32 and rounded once to the element type: the gradient of an input that
// several groups of one packed scan call read (a level's write is the source
// key of its outgoing relation edges and the target value of its incoming
// ones), formed in one pass instead of a chain of pairwise adds.  HBM bound:
// n reads and one write per element.
#include <hip/hip_runtime.h>

#include "gpa_common.h"
#include "gpa_hip.h"

namespace gpa {
namespace {

struct SumPack {
  const uint4* src[GPA_SUM_MAX];
  uint4* dst;
  int64_t count;  // 16-byte vectors
  int n;
};

__device__ __forceinline__ void add8(float (&acc)[8], uint4 w, bool bf16) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
  if (bf16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] += __uint_as_float(u[i] << 16);
      acc[2 * i + 1] += __uint_as_float(u[i] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] += __uint_as_float(u[i]);
  }
}

template <bool BF16>
__global__ __launch_bounds__(256) void sum_many(SumPack pk) {
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < pk.count; e += (int64_t)gridDim.x * 256) {
    uint4 w[GPA_SUM_MAX];
#pragma unroll
    for (int j = 0; j < GPA_SUM_MAX; ++j) w[j] = j < pk.n ? pk.src[j][e] : make_uint4(0, 0, 0, 0);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < GPA_SUM_MAX; ++j)
      if (j < pk.n) add8(acc, w[j], BF16);
    uint4 o;
    if (BF16) {
      uint32_t r[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        r[i] = (uint32_t)from_f32<bf16_t>(acc[2 * i]).bits | ((uint32_t)from_f32<bf16_t>(acc[2 * i + 1]).bits << 16);
      o = make_uint4(r[0], r[1], r[2], r[3]);
    } else {
      o = make_uint4(__float_as_uint(acc[0]), __float_as_uint(acc[1]), __float_as_uint(acc[2]),
                     __float_as_uint(acc[3]));
    }
    pk.dst[e] = o;
  }
}

}  // namespace
}  // namespace gpa

extern "C" int gpa_sum_many(void* dst, const void* const* src, int32_t n, int64_t count, int32_t dtype,
                            hipStream_t stream) {
  using namespace gpa;
  if (!dst || !src || n < 1 || n > GPA_SUM_MAX || count < 0)
    return fail(GPA_HIP_EINVAL, "sum many: 1 to GPA_SUM_MAX sources and a destination");
  if (dtype != GPA_DTYPE_F32 && dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "sum many: dtype");
  const int64_t per = dtype == GPA_DTYPE_BF16 ? 8 : 4;
  if (count % per || (uintptr_t)dst % 16) return fail(GPA_HIP_EINVAL, "sum many: 16-byte aligned whole vectors");
  SumPack pk{};
  for (int j = 0; j < n; ++j) {
    if (!src[j] || (uintptr_t)src[j] % 16) return fail(GPA_HIP_EINVAL, "sum many: 16-byte aligned sources");
    pk.src[j] = static_cast<const uint4*>(src[j]);
  }
  pk.dst = static_cast<uint4*>(dst);
  pk.count = count / per;
  pk.n = n;
  if (!pk.count) return GPA_HIP_OK;
  const int64_t blocks = (pk.count + 255) / 256;
  const dim3 grid((unsigned)(blocks < 2048 ? blocks : 2048));
  if (dtype == GPA_DTYPE_BF16) hipLaunchKernelGGL(sum_many<true>, grid, dim3(256), 0, stream, pk);
  else hipLaunchKernelGGL(sum_many<false>, grid, dim3(256), 0, stream, pk);
  return check_launch("gpa_sum_many");
}
