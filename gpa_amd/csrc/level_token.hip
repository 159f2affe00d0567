// One-token level write and residual (inference decode): reference
// src/gpa/attention.py:314-329 (_block_segment) and :190-194 (_residual) for a
// single token of every stream, from the block snapshots A^ [Dk][M] and
// B^ [M][Dv]:
//
//   w = softmax(u(key) A^), rounded to the activation type (the write)
//   key'   = key   - eta0 round(A^ w)
//   value' = value - eta1 round(w^T B^)
//
// One 256-thread workgroup per stream.  The logits and w^T B^ are column sums
// over rows (threads own a column; when the width is below 256 the rows are
// split between thread groups and the partial sums meet in LDS); A^ w is a
// row dot product per wave, eight rows at a time.  HBM bound: A^ is read
// twice (the second time mostly from cache), B^ once.
#include "gdn_common.h"

namespace gpa {
namespace {

constexpr int QNT = 256;  // threads per workgroup; every width is at most 256

template <typename E>
__global__ __launch_bounds__(QNT) void level_token(gpa_level_problem p) {
  __shared__ float uk[QNT], wf[QNT], zs[QNT], zp[QNT], rks[QNT];
  __shared__ float red[4], soft[2];
  const int s = blockIdx.x, b = s / p.heads, h = s - b * p.heads;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int Dk = p.key_dim, Dv = p.value_dim, M = p.slots;
  const float* A = p.a_first + (int64_t)b * p.a_first_sb + (int64_t)h * Dk * M;   // [Dk][M]
  const float* Bh = p.b_first + (int64_t)b * p.b_first_sb + (int64_t)h * M * Dv;  // [M][Dv]
  const E* key = reinterpret_cast<const E*>(p.key.ptr) + op_base(p.key, b, h);
  const E* val = reinterpret_cast<const E*>(p.value.ptr) + op_base(p.value, b, h);
  const float eta0 = p.eta[2 * h], eta1 = p.eta[2 * h + 1];

  // u(key) = key / max(||key||, 1e-6) in float32, rounded to the activation type.
  const float xk = t < Dk ? to_f32(key[t < Dk ? t : 0]) : 0.f;
  const float sk = sum64(xk * xk);
  if (lane == 0) red[wave] = sk;
  lds_barrier();
  const float nk = fmaxf(sqrtf(red[0] + red[1] + red[2] + red[3]), 1e-6f);
  if (t < Dk) uk[t] = round_as<E>(xk / nk);
  lds_barrier();

  // Logits z[m] = sum_k u(key)[k] A^[k][m]: thread (part, col), rows part + P i.
  {
    const int P = QNT / M, col = t % M, part = t / M;
    float z = 0.f;
    if (part < P) {
#pragma unroll 8
      for (int k = part; k < Dk; k += P) z += uk[k] * A[(int64_t)k * M + col];
    }
    zp[t] = z;
    lds_barrier();
    if (t < M) {
      float zt = 0.f;
      for (int q = 0; q < P; ++q) zt += zp[q * M + t];
      zs[t] = zt;
    }
    lds_barrier();
  }

  // Softmax over the M logits; the write is rounded to the activation type.
  if (wave == 0) {
    float mx = -INFINITY;
    for (int m = lane; m < M; m += 64) mx = fmaxf(mx, zs[m]);
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    float sm = 0.f;
    for (int m = lane; m < M; m += 64) sm += expf(zs[m] - mx);
    sm = sum64(sm);
    if (lane == 0) {
      soft[0] = mx;
      soft[1] = sm;
    }
  }
  lds_barrier();
  if (t < M) {
    const float w = round_as<E>(expf(zs[t] - soft[0]) / soft[1]);
    wf[t] = w;
    reinterpret_cast<E*>(p.write.ptr)[op_base(p.write, b, h) + t] = from_f32<E>(w);
  }
  lds_barrier();

  // rk[k] = sum_m A^[k][m] w[m]: wave `wave` takes rows wave + 4 r, eight rows
  // per pass with every load of the pass issued before the sums.
  for (int k0 = wave; k0 < Dk; k0 += 4 * 8) {
    float acc[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) acc[r] = 0.f;
    for (int m = lane; m < M; m += 64) {
      const float w = wf[m];
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int k = k0 + 4 * r;
        acc[r] += A[(int64_t)(k < Dk ? k : 0) * M + m] * w;
      }
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const float v = sum64(acc[r]);
      const int k = k0 + 4 * r;
      if (lane == 0 && k < Dk) rks[k] = v;
    }
  }

  // rv[v] = sum_m w[m] B^[m][v]: thread (part, col), rows part + P2 i.
  {
    const int P2 = QNT / Dv, col = t % Dv, part = t / Dv;
    float acc = 0.f;
    if (part < P2) {
#pragma unroll 8
      for (int m = part; m < M; m += P2) acc += wf[m] * Bh[(int64_t)m * Dv + col];
    }
    zp[t] = acc;
  }
  lds_barrier();
  if (t < Dv) {
    const int P2 = QNT / Dv;
    float rv = 0.f;
    for (int q = 0; q < P2; ++q) rv += zp[q * Dv + t];
    const float v = to_f32(val[t]);
    reinterpret_cast<E*>(p.value_out.ptr)[op_base(p.value_out, b, h) + t] = from_f32<E>(v - eta1 * round_as<E>(rv));
  }
  if (t < Dk) {
    reinterpret_cast<E*>(p.key_out.ptr)[op_base(p.key_out, b, h) + t] =
        from_f32<E>(xk - eta0 * round_as<E>(rks[t]));
  }
}

}  // namespace
}  // namespace gpa

extern "C" int gpa_level_token_forward(const gpa_level_problem* problem, hipStream_t stream) {
  using namespace gpa;
  if (!problem) return fail(GPA_HIP_EINVAL, "level token: null problem");
  const gpa_level_problem& p = *problem;
  if (p.tokens != 1) return fail(GPA_HIP_EINVAL, "level token: needs tokens == 1");
  if (p.batch < 1 || p.heads < 1) return fail(GPA_HIP_EINVAL, "level token: empty shape");
  if (p.key_dim < 1 || p.key_dim > QNT || p.value_dim < 1 || p.value_dim > QNT || p.slots < 1 || p.slots > QNT)
    return fail(GPA_HIP_EUNSUPPORTED, "level token: key, value and slot widths must be in [1, 256]");
  if (p.dtype != GPA_DTYPE_F32 && p.dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "level token: dtype");
  if (!p.key.ptr || !p.value.ptr || !p.a_first || !p.b_first || !p.eta || !p.write.ptr || !p.key_out.ptr ||
      !p.value_out.ptr)
    return fail(GPA_HIP_EINVAL, "level token: null pointer (the snapshots a_first and b_first are required)");
  const dim3 grid((unsigned)((int64_t)p.batch * p.heads));
  if (p.dtype == GPA_DTYPE_BF16) hipLaunchKernelGGL(level_token<bf16_t>, grid, dim3(QNT), 0, stream, p);
  else hipLaunchKernelGGL(level_token<float>, grid, dim3(QNT), 0, stream, p);
  return check_launch("gpa_level_token_forward");
}
