// Element-wise glue of the inference path, one launch each where the device
// ops of the schedule take several: the gate nonlinearities of a level, the
// one-token counts / base logits / local read distribution of a level, and the
// output mix over the levels.  Each follows the reference's float32 arithmetic
// and its rounding to the activation type.
#include <hip/hip_runtime.h>

#include "glue_rows.h"

namespace gpa {
namespace {

// reference attention.py:161-174 after the gate-input product.
template <typename E>
__global__ void gate_act(gpa_gate_problem p) {
  const int n = p.batch * p.tokens * p.heads;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int h = i % p.heads, bt = i / p.heads, t = bt % p.tokens, b = bt / p.tokens;
  float raw[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) raw[c] = act_at<E>(p.raw, b, t, h, c);
  gate_row(p, h, i, raw);
}

// Backward of the gate nonlinearities (the autograd of attention.py:166-174):
// x = float(raw) + bias; d decay / dx = -decay_scale softplus'(x) where
// softplus(x) <= 10 (the clamp passes its bound), softplus' = z / (z + 1),
// z = e^x (1 above the threshold 20); d strength / dx = beta_max s (1 - s).
// draw is the float32 gradient rounded to the activation type (the cast's
// backward); dbias gets per-workgroup partial sums over its rows (LDS atomics
// by head).
template <typename E>
__global__ __launch_bounds__(256) void gate_act_bwd(gpa_gate_problem p, gpa_gate_grads g) {
  __shared__ float db[GPA_GATE_MAX_HEADS * 4];
  const int H = p.heads;
  for (int i = threadIdx.x; i < 4 * H; i += 256) db[i] = 0.f;
  __syncthreads();
  const int64_t n = (int64_t)p.batch * p.tokens * H;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) {
    const int h = (int)(i % H);
    const int64_t bt = i / H;
    const int t = (int)(bt % p.tokens), b = (int)(bt / p.tokens);
    float x[4], d[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) x[c] = act_at<E>(p.raw, b, t, h, c) + p.bias[4 * h + c];
    const float gi = g.dg_in ? g.dg_in[i] : 0.f, bi = g.db_in ? g.db_in[i] : 0.f;
    const float go = g.dg_out ? g.dg_out[i] : 0.f, bo = g.db_out ? g.db_out[i] : 0.f;
#pragma unroll
    for (int c = 0; c < 4; c += 2) {  // decays: channels 0 and 2
      const float dg = c == 0 ? gi : go;
      const float sp = softplus20(x[c]);
      const float z = expf(x[c]);
      const float dsp = x[c] > 20.f ? 1.f : z / (z + 1.f);
      d[c] = sp <= 10.f ? -(dg * p.decay_scale) * dsp : 0.f;
    }
#pragma unroll
    for (int c = 1; c < 4; c += 2) {  // strengths: channels 1 and 3
      const float dbv = (c == 1 ? bi : bo) * p.beta_max;
      const float sg = sigmoid1(x[c]);
      d[c] = dbv * (1.f - sg) * sg;
    }
    E* dr = reinterpret_cast<E*>(g.draw.ptr) + (int64_t)b * g.draw.sb + (int64_t)t * g.draw.st + (int64_t)h * g.draw.sh;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      dr[c] = from_f32<E>(d[c]);
      atomicAdd(&db[4 * h + c], d[c]);
    }
  }
  __syncthreads();
  for (int k = threadIdx.x; k < 4 * H; k += 256) g.dbias[(int64_t)blockIdx.x * 4 * H + k] = db[k];
}

// One token of one level: n = count0 + write; logits = scale raw + gain
// log1p(n); local = round(softmax(logits)).  One 64-lane wave per (b, h) row.
template <typename E>
__global__ __launch_bounds__(256) void token_logits(gpa_token_logits_problem p) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= p.batch * p.heads) return;
  token_logits_row<E>(p, row / p.heads, row % p.heads, lane);
}

// Several levels' token logits in one launch: workgroups wg0[i] .. wg0[i+1]-1
// take problem i (four rows each), read from the kernel arguments.
struct LogitsPack {
  int n;
  int wg0[GPA_TOKEN_LOGITS_MAX_PACK];
  gpa_token_logits_problem p[GPA_TOKEN_LOGITS_MAX_PACK];
};

template <typename E>
__global__ __launch_bounds__(256) void token_logits_pack(LogitsPack pk) {
  typedef const __attribute__((address_space(4))) LogitsPack* KernargPtr;
  const KernargPtr kp = (KernargPtr)__builtin_amdgcn_kernarg_segment_ptr();
  int pi = 0;
#pragma unroll 1
  for (int i = 1; i < kp->n; ++i)
    if ((int)blockIdx.x >= kp->wg0[i]) pi = i;
  gpa_token_logits_problem p;
  kernarg_copy(p, &kp->p[pi]);
  const int row = ((int)blockIdx.x - kp->wg0[pi]) * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= p.batch * p.heads) return;
  token_logits_row<E>(p, row / p.heads, row % p.heads, lane);
}

// out = round(sum_j w[j,h] read_j), summed in level order (attention.py:340-341).
template <typename E>
__global__ void output_mix(gpa_mix_problem p) {
#pragma clang fp contract(off)
  const int64_t n = (int64_t)p.batch * p.tokens * p.heads * p.value_dim;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int d = (int)(i % p.value_dim);
  int64_t r = i / p.value_dim;
  const int h = (int)(r % p.heads);
  r /= p.heads;
  const int t = (int)(r % p.tokens), b = (int)(r / p.tokens);
  float acc = 0.f;
  for (int j = 0; j < p.levels; ++j) {  // a product and a sum per level, rounded separately (no contraction)
    const float prod = p.weights[j * p.heads + h] * act_at<E>(p.read[j], b, t, h, d);
    acc = acc + prod;
  }
  reinterpret_cast<E*>(p.out.ptr)[(int64_t)b * p.out.sb + (int64_t)t * p.out.st + (int64_t)h * p.out.sh + d] =
      from_f32<E>(acc);
}

// Backward of output_mix over tiles of MIX_ROWS tokens: dread_j = round(w[j,h]
// dout) (the gradient of w x in float32, cast to the reads' type) and the
// tile's partial sums of dw[j,h] = sum dout read_j.  Thread t owns the 16-byte
// column vectors t, t + 256 of a token's H*V values (one head each: V is a
// whole number of vectors), so its partial sums stay in registers until one
// LDS reduction; the loads of four rows are issued before their use.
constexpr int MIX_ROWS = 32, MIX_VECS = 2, MIX_UNROLL = 4;

template <typename E>
struct MixVec {
  static constexpr int N = 16 / sizeof(E);  // elements per 16-byte vector
};

template <typename E>
__device__ __forceinline__ void unpack16(uint4 w, float (&x)[MixVec<E>::N]) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
  if constexpr (sizeof(E) == 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(u[i] << 16);
      x[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = __uint_as_float(u[i]);
  }
}

template <typename E>
__device__ __forceinline__ uint4 pack16(const float (&x)[MixVec<E>::N]) {
  uint32_t u[4];
  if constexpr (sizeof(E) == 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      u[i] = (uint32_t)from_f32<bf16_t>(x[2 * i]).bits | ((uint32_t)from_f32<bf16_t>(x[2 * i + 1]).bits << 16);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = __float_as_uint(x[i]);
  }
  return make_uint4(u[0], u[1], u[2], u[3]);
}

__device__ __forceinline__ int64_t mix_at(const gpa_operand& o, int b, int t, int h, int d) {
  return (int64_t)b * o.sb + (int64_t)t * o.st + (int64_t)h * o.sh + d;
}

template <typename E>
__global__ __launch_bounds__(256) void output_mix_bwd(gpa_mix_problem p, gpa_mix_grads g) {
  constexpr int N = MixVec<E>::N, LMAX = GPA_DECODE_MAX_LEVELS;
  __shared__ float dw[LMAX * GPA_MIX_MAX_HEADS];
  const int tid = threadIdx.x, H = p.heads, V = p.value_dim, NV = H * V / N, L = p.levels;
  for (int i = tid; i < L * H; i += 256) dw[i] = 0.f;
  __syncthreads();
  float acc[MIX_VECS][LMAX];
  float wv[MIX_VECS][LMAX];
  int hv[MIX_VECS], dv[MIX_VECS];
#pragma unroll
  for (int ci = 0; ci < MIX_VECS; ++ci) {
    const int c = (tid + 256 * ci) * N, cc = c < H * V ? c : 0;
    hv[ci] = cc / V;
    dv[ci] = cc % V;
#pragma unroll
    for (int j = 0; j < LMAX; ++j) {
      acc[ci][j] = 0.f;
      wv[ci][j] = j < L ? p.weights[j * H + hv[ci]] : 0.f;
    }
  }
  const int64_t rows = (int64_t)p.batch * p.tokens, r0 = (int64_t)blockIdx.x * MIX_ROWS;
  for (int64_t rb = r0; rb < r0 + MIX_ROWS; rb += MIX_UNROLL) {
#pragma unroll
    for (int ci = 0; ci < MIX_VECS; ++ci) {
      if (tid + 256 * ci >= NV) continue;
      uint4 go[MIX_UNROLL], rd[MIX_UNROLL][LMAX];
      // every load of the four rows first (clamped to a valid row), then the math
#pragma unroll
      for (int u = 0; u < MIX_UNROLL; ++u) {
        const int64_t r = rb + u < rows ? rb + u : rows - 1;
        const int b = (int)(r / p.tokens), t = (int)(r % p.tokens);
        go[u] = *reinterpret_cast<const uint4*>(reinterpret_cast<const E*>(g.dout.ptr) +
                                                mix_at(g.dout, b, t, hv[ci], dv[ci]));
#pragma unroll
        for (int j = 0; j < LMAX; ++j)
          rd[u][j] = j < L ? *reinterpret_cast<const uint4*>(reinterpret_cast<const E*>(p.read[j].ptr) +
                                                            mix_at(p.read[j], b, t, hv[ci], dv[ci]))
                           : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < MIX_UNROLL; ++u) {
        if (rb + u >= rows || rb + u >= r0 + MIX_ROWS) continue;
        const int64_t r = rb + u;
        const int b = (int)(r / p.tokens), t = (int)(r % p.tokens);
        float gx[N];
        unpack16<E>(go[u], gx);
#pragma unroll
        for (int j = 0; j < LMAX; ++j) {
          if (j >= L) break;
          float x[N], y[N];
          unpack16<E>(rd[u][j], x);
#pragma unroll
          for (int e = 0; e < N; ++e) {
            y[e] = gx[e] * wv[ci][j];
            acc[ci][j] += gx[e] * x[e];
          }
          *reinterpret_cast<uint4*>(reinterpret_cast<E*>(g.dread[j].ptr) + mix_at(g.dread[j], b, t, hv[ci], dv[ci])) =
              pack16<E>(y);
        }
      }
    }
  }
#pragma unroll
  for (int ci = 0; ci < MIX_VECS; ++ci) {
    if (tid + 256 * ci >= NV) continue;
#pragma unroll
    for (int j = 0; j < LMAX; ++j)
      if (j < L) atomicAdd(&dw[j * H + hv[ci]], acc[ci][j]);
  }
  __syncthreads();
  for (int i = tid; i < L * H; i += 256) g.dweights[(int64_t)blockIdx.x * L * H + i] = dw[i];
}

// output_mix over 16-byte vectors (V a whole number of vectors, aligned rows):
// thread e handles vector e of the [B*T][H*V] output.
template <typename E>
__global__ __launch_bounds__(256) void output_mix_vec(gpa_mix_problem p) {
#pragma clang fp contract(off)
  constexpr int N = MixVec<E>::N;
  const int H = p.heads, V = p.value_dim, NV = H * V / N;
  const int64_t n = (int64_t)p.batch * p.tokens * NV;
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  const int64_t r = e / NV;
  const int c = (int)(e % NV) * N, h = c / V, d = c % V;
  const int b = (int)(r / p.tokens), t = (int)(r % p.tokens);
  uint4 w[GPA_DECODE_MAX_LEVELS];
#pragma unroll
  for (int j = 0; j < GPA_DECODE_MAX_LEVELS; ++j)
    w[j] = j < p.levels ? *reinterpret_cast<const uint4*>(reinterpret_cast<const E*>(p.read[j].ptr) +
                                                         mix_at(p.read[j], b, t, h, d))
                        : make_uint4(0, 0, 0, 0);
  float acc[N];
#pragma unroll
  for (int i = 0; i < N; ++i) acc[i] = 0.f;
#pragma unroll
  for (int j = 0; j < GPA_DECODE_MAX_LEVELS; ++j) {
    if (j >= p.levels) break;
    float x[N];
    unpack16<E>(w[j], x);
    const float wj = p.weights[j * H + h];
#pragma unroll
    for (int i = 0; i < N; ++i) {  // a product and a sum per level, rounded separately
      const float prod = wj * x[i];
      acc[i] = acc[i] + prod;
    }
  }
  *reinterpret_cast<uint4*>(reinterpret_cast<E*>(p.out.ptr) + mix_at(p.out, b, t, h, d)) = pack16<E>(acc);
}

// Row softmax of float32 logits rounded to E (the local read distribution,
// attention.py:330: softmax(logits).to(dtype)), one wave per row of m <= 1024
// values (16 per lane), and its backward dx = s (dy - sum s dy) with s the
// float32 softmax recomputed from the logits.
template <int PER>
__device__ __forceinline__ void smx_row(const float* x, int m, int lane, float (&s)[PER]) {
  float v[PER], mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int c = lane + 64 * i;
    v[i] = x[c < m ? c : 0];
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    if (lane + 64 * i >= m) v[i] = -INFINITY;
    mx = fmaxf(mx, v[i]);
  }
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    s[i] = lane + 64 * i < m ? expf(v[i] - mx) : 0.f;
    sum += s[i];
  }
  sum = sum64(sum);
#pragma unroll
  for (int i = 0; i < PER; ++i) s[i] = s[i] / sum;
}

// PER values per lane: m <= 64 PER.
template <typename E, int PER>
__global__ __launch_bounds__(256) void row_softmax_fwd(const float* x, E* y, int64_t rows, int m) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  float s[PER];
  smx_row<PER>(x + row * m, m, lane, s);
#pragma unroll
  for (int i = 0; i < PER; ++i)
    if (lane + 64 * i < m) y[row * m + lane + 64 * i] = from_f32<E>(s[i]);
}

template <typename E, int PER>
__global__ __launch_bounds__(256) void row_softmax_bwd(const float* x, const E* dy, float* dx, int64_t rows, int m) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  float g[PER], s[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int c = lane + 64 * i;
    g[i] = to_f32(dy[row * m + (c < m ? c : 0)]);
  }
  smx_row<PER>(x + row * m, m, lane, s);
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) dot += lane + 64 * i < m ? s[i] * g[i] : 0.f;
  dot = sum64(dot);
#pragma unroll
  for (int i = 0; i < PER; ++i)
    if (lane + 64 * i < m) dx[row * m + lane + 64 * i] = s[i] * (g[i] - dot);
}

// Launches KERNEL<E, PER> with the smallest PER in {1, 2, 4, 8, 16} that covers m.
#define GPA_SMX_LAUNCH(KERNEL, E, m, grid, ...)                                                \
  do {                                                                                        \
    if ((m) <= 64) hipLaunchKernelGGL((KERNEL<E, 1>), grid, dim3(256), 0, __VA_ARGS__);       \
    else if ((m) <= 128) hipLaunchKernelGGL((KERNEL<E, 2>), grid, dim3(256), 0, __VA_ARGS__); \
    else if ((m) <= 256) hipLaunchKernelGGL((KERNEL<E, 4>), grid, dim3(256), 0, __VA_ARGS__); \
    else if ((m) <= 512) hipLaunchKernelGGL((KERNEL<E, 8>), grid, dim3(256), 0, __VA_ARGS__); \
    else hipLaunchKernelGGL((KERNEL<E, 16>), grid, dim3(256), 0, __VA_ARGS__);                \
  } while (0)

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

namespace gpa {
namespace {
int check_token_logits(const gpa_token_logits_problem* p) {
  if (!p || !p->raw.ptr || !p->write.ptr || !p->count0 || !p->gain || !p->scale || !p->logits || !p->count ||
      !p->local)
    return fail(GPA_HIP_EINVAL, "token logits: null pointer");
  if (p->batch < 1 || p->heads < 1) return fail(GPA_HIP_EINVAL, "token logits: empty shape");
  if ((int64_t)p->batch * p->heads > 0x7fffffff) return fail(GPA_HIP_EUNSUPPORTED, "token logits: too many rows");
  if (p->slots < 1 || p->slots > GPA_TOKEN_LOGITS_MAX_SLOTS)
    return fail(GPA_HIP_EUNSUPPORTED, "token logits: slots must be in [1, 256]");
  if (p->dtype != GPA_DTYPE_F32 && p->dtype != GPA_DTYPE_BF16)
    return fail(GPA_HIP_EUNSUPPORTED, "token logits: dtype");
  return GPA_HIP_OK;
}
}  // namespace
}  // namespace gpa

extern "C" int gpa_token_logits_forward(const gpa_token_logits_problem* p, hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_token_logits(p)) return rc;
  const int rows = p->batch * p->heads;
  const dim3 grid((rows + 3) / 4), block(256);
  if (p->dtype == GPA_DTYPE_BF16)
    hipLaunchKernelGGL(token_logits<bf16_t>, grid, block, 0, stream, *p);
  else
    hipLaunchKernelGGL(token_logits<float>, grid, block, 0, stream, *p);
  return check_launch("gpa_token_logits_forward");
}

extern "C" int gpa_token_logits_many(const gpa_token_logits_problem* problems, int32_t n, hipStream_t stream) {
  using namespace gpa;
  if (n < 0 || n > GPA_TOKEN_LOGITS_MAX_PACK) return fail(GPA_HIP_EINVAL, "token logits: 0 to 8 problems per call");
  if (n == 0) return GPA_HIP_OK;
  if (!problems) return fail(GPA_HIP_EINVAL, "token logits: null problems");
  LogitsPack pk{};
  int64_t wgs = 0;
  for (int i = 0; i < n; ++i) {
    const gpa_token_logits_problem& p = problems[i];
    if (int rc = check_token_logits(&p)) return rc;
    if (p.dtype != problems[0].dtype) return fail(GPA_HIP_EINVAL, "token logits: one dtype per call");
    pk.p[i] = p;
    pk.wg0[i] = (int)wgs;
    wgs += ((int64_t)p.batch * p.heads + 3) / 4;
  }
  pk.n = n;
  if (wgs > 0x7fffffff) return fail(GPA_HIP_EUNSUPPORTED, "token logits: too many rows");
  if (problems[0].dtype == GPA_DTYPE_BF16)
    hipLaunchKernelGGL(token_logits_pack<bf16_t>, dim3((unsigned)wgs), dim3(256), 0, stream, pk);
  else
    hipLaunchKernelGGL(token_logits_pack<float>, dim3((unsigned)wgs), dim3(256), 0, stream, pk);
  return check_launch("gpa_token_logits_many");
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
  const int vec = p->dtype == GPA_DTYPE_BF16 ? 8 : 4;  // elements per 16-byte vector
  auto aligned = [&](const gpa_operand& o) {
    return (uintptr_t)o.ptr % 16 == 0 && o.sb % vec == 0 && o.st % vec == 0 && o.sh % vec == 0;
  };
  bool vectors = p->value_dim % vec == 0 && aligned(p->out);
  for (int j = 0; j < p->levels; ++j) vectors = vectors && aligned(p->read[j]);
  const dim3 block(256);
  if (vectors) {
    const dim3 grid((unsigned)((n / vec + 255) / 256));
    if (p->dtype == GPA_DTYPE_BF16)
      hipLaunchKernelGGL(output_mix_vec<bf16_t>, grid, block, 0, stream, *p);
    else
      hipLaunchKernelGGL(output_mix_vec<float>, grid, block, 0, stream, *p);
  } else {
    const dim3 grid((unsigned)((n + 255) / 256));
    if (p->dtype == GPA_DTYPE_BF16)
      hipLaunchKernelGGL(output_mix<bf16_t>, grid, block, 0, stream, *p);
    else
      hipLaunchKernelGGL(output_mix<float>, grid, block, 0, stream, *p);
  }
  return check_launch("gpa_output_mix_forward");
}

namespace gpa {
namespace {

// Up to GPA_COPY_MAX buffers copied in one launch (grid.y = buffer), 16 bytes
// per thread per step; every buffer and size is a multiple of 16 bytes.
struct CopyPack {
  const uint4* src[GPA_COPY_MAX];
  uint4* dst[GPA_COPY_MAX];
  int64_t count[GPA_COPY_MAX];
};

__global__ __launch_bounds__(256) void copy_many(CopyPack pk) {
  const int i = blockIdx.y;  // uniform: selects, not a dynamic index into the argument
  const uint4* src = i == 0 ? pk.src[0] : i == 1 ? pk.src[1] : i == 2 ? pk.src[2] : pk.src[3];
  uint4* dst = i == 0 ? pk.dst[0] : i == 1 ? pk.dst[1] : i == 2 ? pk.dst[2] : pk.dst[3];
  const int64_t n = i == 0 ? pk.count[0] : i == 1 ? pk.count[1] : i == 2 ? pk.count[2] : pk.count[3];
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) dst[e] = src[e];
}

}  // namespace
}  // namespace gpa

extern "C" int gpa_copy_many(void* const* dst, const void* const* src, const int64_t* bytes, int32_t n,
                             hipStream_t stream) {
  using namespace gpa;
  if (!dst || !src || !bytes || n < 1 || n > GPA_COPY_MAX)
    return fail(GPA_HIP_EINVAL, "copy many: 1 to GPA_COPY_MAX buffers");
  CopyPack pk{};
  int64_t most = 0;
  for (int i = 0; i < n; ++i) {
    if (bytes[i] < 0 || bytes[i] % 16 || (bytes[i] && (!dst[i] || !src[i])) || (uintptr_t)dst[i] % 16 ||
        (uintptr_t)src[i] % 16)
      return fail(GPA_HIP_EINVAL, "copy many: buffers and sizes must be multiples of 16 bytes");
    pk.src[i] = static_cast<const uint4*>(src[i]);
    pk.dst[i] = static_cast<uint4*>(dst[i]);
    pk.count[i] = bytes[i] / 16;
    most = pk.count[i] > most ? pk.count[i] : most;
  }
  if (!most) return GPA_HIP_OK;
  const int64_t blocks = (most + 255) / 256;
  hipLaunchKernelGGL(copy_many, dim3((unsigned)(blocks < 1024 ? blocks : 1024), (unsigned)n), dim3(256), 0, stream, pk);
  return check_launch("gpa_copy_many");
}

extern "C" int gpa_output_mix_backward(const gpa_mix_problem* p, const gpa_mix_grads* g, hipStream_t stream) {
  using namespace gpa;
  if (!p || !g || !p->weights || !g->dout.ptr || !g->dweights) return fail(GPA_HIP_EINVAL, "output mix backward: null pointer");
  if (p->levels < 1 || p->levels > GPA_DECODE_MAX_LEVELS)
    return fail(GPA_HIP_EINVAL, "output mix backward: 1 to 4 levels");
  for (int j = 0; j < p->levels; ++j)
    if (!p->read[j].ptr || !g->dread[j].ptr) return fail(GPA_HIP_EINVAL, "output mix backward: null read");
  if (p->batch < 1 || p->tokens < 1 || p->heads < 1 || p->value_dim < 1)
    return fail(GPA_HIP_EINVAL, "output mix backward: empty shape");
  const int vec = p->dtype == GPA_DTYPE_BF16 ? 8 : 4;  // elements per 16-byte vector
  if (p->heads > GPA_MIX_MAX_HEADS || (int64_t)p->heads * p->value_dim > 256 * MIX_VECS * vec)
    return fail(GPA_HIP_EUNSUPPORTED, "output mix backward: heads <= GPA_MIX_MAX_HEADS, heads*value_dim <= 512 vectors");
  auto aligned = [&](const gpa_operand& o) {
    return (uintptr_t)o.ptr % 16 == 0 && o.sb % vec == 0 && o.st % vec == 0 && o.sh % vec == 0;
  };
  bool ok = p->value_dim % vec == 0 && aligned(g->dout);
  for (int j = 0; j < p->levels; ++j) ok = ok && aligned(p->read[j]) && aligned(g->dread[j]);
  if (!ok) return fail(GPA_HIP_EINVAL, "output mix backward: 16-byte aligned rows, value_dim a whole number of vectors");
  if (p->dtype != GPA_DTYPE_F32 && p->dtype != GPA_DTYPE_BF16)
    return fail(GPA_HIP_EUNSUPPORTED, "output mix backward: dtype");
  const int64_t tiles = ((int64_t)p->batch * p->tokens + MIX_ROWS - 1) / MIX_ROWS;
  if (tiles > 0x7fffffff) return fail(GPA_HIP_EINVAL, "output mix backward: too many tokens");
  if (p->dtype == GPA_DTYPE_BF16)
    hipLaunchKernelGGL(output_mix_bwd<bf16_t>, dim3((unsigned)tiles), dim3(256), 0, stream, *p, *g);
  else
    hipLaunchKernelGGL(output_mix_bwd<float>, dim3((unsigned)tiles), dim3(256), 0, stream, *p, *g);
  return check_launch("gpa_output_mix_backward");
}

extern "C" int gpa_row_softmax_forward(const float* x, void* y, int64_t rows, int32_t m, int32_t dtype,
                                       hipStream_t stream) {
  using namespace gpa;
  if (!x || !y || rows < 0 || m < 1 || m > 1024) return fail(GPA_HIP_EINVAL, "row softmax: 1 <= m <= 1024");
  if (dtype != GPA_DTYPE_F32 && dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "row softmax: dtype");
  if (!rows) return GPA_HIP_OK;
  if ((rows + 3) / 4 > 0x7fffffff) return fail(GPA_HIP_EINVAL, "row softmax: too many rows");
  const dim3 grid((unsigned)((rows + 3) / 4));
  if (dtype == GPA_DTYPE_BF16)
    GPA_SMX_LAUNCH(row_softmax_fwd, bf16_t, m, grid, stream, x, static_cast<bf16_t*>(y), rows, m);
  else
    GPA_SMX_LAUNCH(row_softmax_fwd, float, m, grid, stream, x, static_cast<float*>(y), rows, m);
  return check_launch("gpa_row_softmax_forward");
}

extern "C" int gpa_row_softmax_backward(const float* x, const void* dy, float* dx, int64_t rows, int32_t m,
                                        int32_t dtype, hipStream_t stream) {
  using namespace gpa;
  if (!x || !dy || !dx || rows < 0 || m < 1 || m > 1024)
    return fail(GPA_HIP_EINVAL, "row softmax backward: 1 <= m <= 1024");
  if (dtype != GPA_DTYPE_F32 && dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "row softmax: dtype");
  if (!rows) return GPA_HIP_OK;
  if ((rows + 3) / 4 > 0x7fffffff) return fail(GPA_HIP_EINVAL, "row softmax: too many rows");
  const dim3 grid((unsigned)((rows + 3) / 4));
  if (dtype == GPA_DTYPE_BF16)
    GPA_SMX_LAUNCH(row_softmax_bwd, bf16_t, m, grid, stream, x, static_cast<const bf16_t*>(dy), dx, rows, m);
  else
    GPA_SMX_LAUNCH(row_softmax_bwd, float, m, grid, stream, x, static_cast<const float*>(dy), dx, rows, m);
  return check_launch("gpa_row_softmax_backward");
}

extern "C" int gpa_gate_act_backward(const gpa_gate_problem* p, const gpa_gate_grads* g, hipStream_t stream) {
  using namespace gpa;
  if (!p || !g || !p->raw.ptr || !p->bias || !g->draw.ptr || !g->dbias) return fail(GPA_HIP_EINVAL, "gates backward: null pointer");
  if (p->batch < 1 || p->tokens < 1 || p->heads < 1) return fail(GPA_HIP_EINVAL, "gates backward: empty shape");
  if (p->heads > GPA_GATE_MAX_HEADS) return fail(GPA_HIP_EUNSUPPORTED, "gates backward: heads <= GPA_GATE_MAX_HEADS");
  if (p->dtype != GPA_DTYPE_F32 && p->dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "gates: dtype");
  const int64_t n = (int64_t)p->batch * p->tokens * p->heads;
  if ((n + 255) / 256 > 0x7fffffff) return fail(GPA_HIP_EUNSUPPORTED, "gates backward: too many rows");
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  if (p->dtype == GPA_DTYPE_BF16)
    hipLaunchKernelGGL(gate_act_bwd<bf16_t>, grid, block, 0, stream, *p, *g);
  else
    hipLaunchKernelGGL(gate_act_bwd<float>, grid, block, 0, stream, *p, *g);
  return check_launch("gpa_gate_act_backward");
}
