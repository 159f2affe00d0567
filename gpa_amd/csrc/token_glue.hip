// Element-wise glue of the inference path, one launch each where the device
// ops of the schedule take several: the gate nonlinearities of a level, the
// one-token counts / base logits / local read distribution of a level, and the
// output mix over the levels.  Each follows the reference's float32 arithmetic
// and its rounding to the activation type.
#include <hip/hip_runtime.h>

#include "gdn_common.h"

namespace gpa {
namespace {

template <typename E>
__device__ __forceinline__ float act_at(const gpa_operand& o, int b, int t, int h, int d) {
  return to_f32(reinterpret_cast<const E*>(o.ptr)[(int64_t)b * o.sb + (int64_t)t * o.st + (int64_t)h * o.sh + d]);
}

// F.softplus with its default threshold 20.
__device__ __forceinline__ float softplus20(float x) { return x > 20.f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float sigmoid1(float x) { return 1.f / (1.f + expf(-x)); }

// reference attention.py:161-174 after the gate-input product.
template <typename E>
__global__ void gate_act(gpa_gate_problem p) {
  const int n = p.batch * p.tokens * p.heads;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int h = i % p.heads, bt = i / p.heads, t = bt % p.tokens, b = bt / p.tokens;
  float x[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) x[c] = act_at<E>(p.raw, b, t, h, c) + p.bias[4 * h + c];
  p.g_in[i] = __fmul_rn(-fminf(softplus20(x[0]), 10.f), p.decay_scale);
  p.b_in[i] = __fmul_rn(p.beta_max, sigmoid1(x[1]));
  p.g_out[i] = __fmul_rn(-fminf(softplus20(x[2]), 10.f), p.decay_scale);
  p.b_out[i] = __fmul_rn(p.beta_max, sigmoid1(x[3]));
}

// One token of one level: n = count0 + write; logits = scale raw + gain
// log1p(n); local = round(softmax(logits)).  One 64-lane wave per (b, h) row.
template <typename E>
__global__ __launch_bounds__(256) void token_logits(gpa_token_logits_problem p) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= p.batch * p.heads) return;
  const int b = row / p.heads, h = row % p.heads, M = p.slots;
  constexpr int PER = GPA_TOKEN_LOGITS_MAX_SLOTS / 64;
  const float* c0 = p.count0 + (int64_t)b * p.count0_sb + (int64_t)h * M;
  const float gain = p.gain[h], scale = p.scale[h];
  float lg[PER], mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int m = lane + 64 * i;
    if (m < M) {
      const float n = c0[m] + act_at<E>(p.write, b, 0, h, m);
      p.count[(int64_t)row * M + m] = n;
      // separate roundings, as the reference's tensor ops (no contraction)
      lg[i] = __fadd_rn(__fmul_rn(scale, act_at<E>(p.raw, b, 0, h, m)), __fmul_rn(gain, log1pf(n)));
      p.logits[(int64_t)row * M + m] = lg[i];
      mx = fmaxf(mx, lg[i]);
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int m = lane + 64 * i;
    lg[i] = m < M ? expf(lg[i] - mx) : 0.f;
    s += lg[i];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
  E* local = reinterpret_cast<E*>(p.local);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int m = lane + 64 * i;
    if (m < M) local[(int64_t)row * M + m] = from_f32<E>(lg[i] / s);
  }
}

// out = round(sum_j w[j,h] read_j), summed in level order (attention.py:340-341).
template <typename E>
__global__ void output_mix(gpa_mix_problem p) {
  const int64_t n = (int64_t)p.batch * p.tokens * p.heads * p.value_dim;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int d = (int)(i % p.value_dim);
  int64_t r = i / p.value_dim;
  const int h = (int)(r % p.heads);
  r /= p.heads;
  const int t = (int)(r % p.tokens), b = (int)(r / p.tokens);
  float acc = 0.f;
  for (int j = 0; j < p.levels; ++j)  // a product and a sum per level, rounded separately (no contraction)
    acc = __fadd_rn(acc, __fmul_rn(p.weights[j * p.heads + h], act_at<E>(p.read[j], b, t, h, d)));
  reinterpret_cast<E*>(p.out.ptr)[(int64_t)b * p.out.sb + (int64_t)t * p.out.st + (int64_t)h * p.out.sh + d] =
      from_f32<E>(acc);
}

}  // namespace
}  // namespace gpa

extern "C" int gpa_gate_act_forward(const gpa_gate_problem* p, hipStream_t stream) {
  using namespace gpa;
  if (!p || !p->raw.ptr || !p->bias || !p->g_in || !p->b_in || !p->g_out || !p->b_out)
    return fail(GPA_HIP_EINVAL, "gates: null pointer");
  if (p->batch < 1 || p->tokens < 1 || p->heads < 1) return fail(GPA_HIP_EINVAL, "gates: empty shape");
  if (p->dtype != GPA_DTYPE_F32 && p->dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "gates: dtype");
  const int64_t n = (int64_t)p->batch * p->tokens * p->heads;
  if (n > 0x7fffffff) return fail(GPA_HIP_EUNSUPPORTED, "gates: too many rows");
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  if (p->dtype == GPA_DTYPE_BF16)
    hipLaunchKernelGGL(gate_act<bf16_t>, grid, block, 0, stream, *p);
  else
    hipLaunchKernelGGL(gate_act<float>, grid, block, 0, stream, *p);
  return check_launch("gpa_gate_act_forward");
}

extern "C" int gpa_token_logits_forward(const gpa_token_logits_problem* p, hipStream_t stream) {
  using namespace gpa;
  if (!p || !p->raw.ptr || !p->write.ptr || !p->count0 || !p->gain || !p->scale || !p->logits || !p->count ||
      !p->local)
    return fail(GPA_HIP_EINVAL, "token logits: null pointer");
  if (p->batch < 1 || p->heads < 1) return fail(GPA_HIP_EINVAL, "token logits: empty shape");
  if (p->slots < 1 || p->slots > GPA_TOKEN_LOGITS_MAX_SLOTS)
    return fail(GPA_HIP_EUNSUPPORTED, "token logits: slots must be in [1, 256]");
  if (p->dtype != GPA_DTYPE_F32 && p->dtype != GPA_DTYPE_BF16)
    return fail(GPA_HIP_EUNSUPPORTED, "token logits: dtype");
  const int rows = p->batch * p->heads;
  const dim3 grid((rows + 3) / 4), block(256);
  if (p->dtype == GPA_DTYPE_BF16)
    hipLaunchKernelGGL(token_logits<bf16_t>, grid, block, 0, stream, *p);
  else
    hipLaunchKernelGGL(token_logits<float>, grid, block, 0, stream, *p);
  return check_launch("gpa_token_logits_forward");
}

extern "C" int gpa_output_mix_forward(const gpa_mix_problem* p, hipStream_t stream) {
  using namespace gpa;
  if (!p || !p->weights || !p->out.ptr) return fail(GPA_HIP_EINVAL, "output mix: null pointer");
  if (p->levels < 1 || p->levels > GPA_DECODE_MAX_LEVELS)
    return fail(GPA_HIP_EINVAL, "output mix: 1 to 4 levels");
  for (int j = 0; j < p->levels; ++j)
    if (!p->read[j].ptr) return fail(GPA_HIP_EINVAL, "output mix: null read");
  if (p->batch < 1 || p->tokens < 1 || p->heads < 1 || p->value_dim < 1)
    return fail(GPA_HIP_EINVAL, "output mix: empty shape");
  if (p->dtype != GPA_DTYPE_F32 && p->dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "output mix: dtype");
  const int64_t n = (int64_t)p->batch * p->tokens * p->heads * p->value_dim;
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  if (p->dtype == GPA_DTYPE_BF16)
    hipLaunchKernelGGL(output_mix<bf16_t>, grid, block, 0, stream, *p);
  else
    hipLaunchKernelGGL(output_mix<float>, grid, block, 0, stream, *p);
  return check_launch("gpa_output_mix_forward");
}
