// Per-row arithmetic of the inference glue, shared by the stand-alone glue
// kernels and the kernels that fuse it (the slot products with their gate
// nonlinearities, the packed token logits), so that both give the same bits.  Each follows the
// reference's float32 arithmetic and its rounding to the activation type.
#pragma once

#include "gdn_common.h"

namespace gpa {

template <typename E>
__device__ __forceinline__ float act_at(const gpa_operand& o, int b, int t, int h, int d) {
  return to_f32(reinterpret_cast<const E*>(o.ptr)[(int64_t)b * o.sb + (int64_t)t * o.st + (int64_t)h * o.sh + d]);
}

// F.softplus with its default threshold 20.
__device__ __forceinline__ float softplus20(float x) { return x > 20.f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float sigmoid1(float x) { return 1.f / (1.f + expf(-x)); }

// The gate nonlinearities of one (token, head) row (reference attention.py:
// 166-174): x = float(raw) + bias; decay -min(softplus(x), 10) * decay_scale,
// strength beta_max sigmoid(x).  `raw` holds the four gate inputs as rounded
// to the activation type; `i` indexes the [B,T,H] outputs.
__device__ __forceinline__ void gate_values(const gpa_gate_problem& p, int h, const float raw[4], float v[4]) {
  float x[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) x[c] = raw[c] + p.bias[4 * h + c];
  v[0] = mul_rn(-fminf(softplus20(x[0]), 10.f), p.decay_scale);
  v[1] = mul_rn(p.beta_max, sigmoid1(x[1]));
  v[2] = mul_rn(-fminf(softplus20(x[2]), 10.f), p.decay_scale);
  v[3] = mul_rn(p.beta_max, sigmoid1(x[3]));
}
__device__ __forceinline__ void gate_row(const gpa_gate_problem& p, int h, int64_t i, const float raw[4]) {
  float v[4];
  gate_values(p, h, raw, v);
  p.g_in[i] = v[0];
  p.b_in[i] = v[1];
  p.g_out[i] = v[2];
  p.b_out[i] = v[3];
}

// One token of one level for the (b, h) row, by one 64-lane wave: n = count0
// + write; logits = scale raw + gain log1p(n); local = round(softmax(logits))
// (attention.py:196-204, :316-323).
template <typename E>
__device__ __forceinline__ void token_logits_row(const gpa_token_logits_problem& p, int b, int h, int lane) {
  const int row = b * p.heads + h, M = p.slots;
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
      lg[i] = add_rn(mul_rn(scale, act_at<E>(p.raw, b, 0, h, m)), mul_rn(gain, log1pf(n)));
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

}  // namespace gpa
