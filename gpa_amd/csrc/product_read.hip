// The product relation read of the route reader (reference attention.py:231-236,
// paper_product_read; relation_marginal adds the marginal term): the base
// logits of one target level take the incoming messages weighted by the edge
// softmax and by the norm of each source level's read distribution,
//   inc  = sum_e (w_e msg_e) n_e,   out = base + (M gexp) inc  [- gexp log1p(counts)],
// after which the route softmax and MLP run in gpa_route_forward.  One wave
// per row (b, t) of one head, lanes along the slots; every product and sum is
// rounded separately in the reference's order (no contraction).
#include <hip/hip_runtime.h>

#include "gdn_common.h"

namespace gpa {
namespace {

constexpr int PNT = 64 * GPA_PRODUCT_ROWS;  // threads per workgroup
constexpr int PPER = GPA_ROUTE_MAX_WIDTH / 64;  // slots per lane

template <typename E>
__device__ __forceinline__ float msg_at(const gpa_operand& o, int b, int t, int h, int m) {
  return to_f32(reinterpret_cast<const E*>(o.ptr)[(int64_t)b * o.sb + (int64_t)t * o.st + (int64_t)h * o.sh + m]);
}
__device__ __forceinline__ float f32_at(const gpa_operand& o, int b, int t, int h, int m) {
  return reinterpret_cast<const float*>(o.ptr)[(int64_t)b * o.sb + (int64_t)t * o.st + (int64_t)h * o.sh + m];
}

template <typename E>
__global__ __launch_bounds__(PNT) void product_fwd(gpa_product_problem p) {
  const int h = blockIdx.y, lane = threadIdx.x & 63, R = p.batch * p.tokens, M = p.slots;
  const int r = blockIdx.x * GPA_PRODUCT_ROWS + (threadIdx.x >> 6);
  if (r >= R) return;
  const int b = r / p.tokens, t = r - b * p.tokens;
  const float gexp = p.gexp[h], mg = mul_rn((float)M, gexp);
  float wn[GPA_ROUTE_MAX_INCOMING], nr[GPA_ROUTE_MAX_INCOMING];
#pragma unroll
  for (int e = 0; e < GPA_ROUTE_MAX_INCOMING; ++e) {
    wn[e] = e < p.incoming ? p.edge_weight[e * p.heads + h] : 0.f;
    nr[e] = e < p.incoming ? f32_at(p.norm[e], b, t, h, 0) : 0.f;
  }
  // every load of the lane before the first use (clamped slot index)
  float x[PPER], mv[GPA_ROUTE_MAX_INCOMING][PPER], cv[PPER];
#pragma unroll
  for (int i = 0; i < PPER; ++i) {
    const int m = lane + 64 * i, mm = m < M ? m : 0;
    x[i] = f32_at(p.base, b, t, h, mm);
#pragma unroll
    for (int e = 0; e < GPA_ROUTE_MAX_INCOMING; ++e)
      mv[e][i] = e < p.incoming ? msg_at<E>(p.msg[e], b, t, h, mm) : 0.f;
    cv[i] = p.marginal ? f32_at(p.counts, b, t, h, mm) : 0.f;
  }
  float* out = p.out + ((int64_t)r * p.heads + h) * M;
#pragma unroll
  for (int i = 0; i < PPER; ++i) {
    const int m = lane + 64 * i;
    if (m >= M) continue;
    float inc = 0.f;
#pragma unroll
    for (int e = 0; e < GPA_ROUTE_MAX_INCOMING; ++e)
      if (e < p.incoming) inc = add_rn(inc, mul_rn(mul_rn(wn[e], mv[e][i]), nr[e]));
    float y = add_rn(x[i], mul_rn(mg, inc));
    if (p.marginal) y = sub_rn(y, mul_rn(gexp, log1pf(cv[i])));
    out[m] = y;
  }
}

template <typename E>
__global__ __launch_bounds__(PNT) void product_bwd(gpa_product_problem p, gpa_product_grads g) {
  __shared__ float part[GPA_PRODUCT_ROWS][2 + GPA_ROUTE_MAX_INCOMING];
  const int h = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6, R = p.batch * p.tokens;
  const int M = p.slots, NI = p.incoming;
  const int r = blockIdx.x * GPA_PRODUCT_ROWS + wave;
  float s_inc = 0.f, s_log = 0.f, s_w[GPA_ROUTE_MAX_INCOMING] = {};
  if (r < R) {
    const int b = r / p.tokens, t = r - b * p.tokens;
    const float gexp = p.gexp[h], mg = mul_rn((float)M, gexp);
    float wn[GPA_ROUTE_MAX_INCOMING], nr[GPA_ROUTE_MAX_INCOMING];
#pragma unroll
    for (int e = 0; e < GPA_ROUTE_MAX_INCOMING; ++e) {
      wn[e] = e < NI ? p.edge_weight[e * p.heads + h] : 0.f;
      nr[e] = e < NI ? f32_at(p.norm[e], b, t, h, 0) : 0.f;
    }
    const int64_t row = (int64_t)r * p.heads + h;
    float dv[PPER], mv[GPA_ROUTE_MAX_INCOMING][PPER], cv[PPER];
#pragma unroll
    for (int i = 0; i < PPER; ++i) {
      const int m = lane + 64 * i, mm = m < M ? m : 0;
      dv[i] = g.dout[row * M + mm];
#pragma unroll
      for (int e = 0; e < GPA_ROUTE_MAX_INCOMING; ++e)
        mv[e][i] = e < NI ? msg_at<E>(p.msg[e], b, t, h, mm) : 0.f;
      cv[i] = p.marginal ? f32_at(p.counts, b, t, h, mm) : 0.f;
    }
    float s_n[GPA_ROUTE_MAX_INCOMING] = {};
#pragma unroll
    for (int i = 0; i < PPER; ++i) {
      const int m = lane + 64 * i;
      if (m >= M) continue;
      const float d = dv[i], dinc = mul_rn(d, mg);
      float inc = 0.f;
#pragma unroll
      for (int e = 0; e < GPA_ROUTE_MAX_INCOMING; ++e)
        if (e < NI) {
          const float wm = mul_rn(wn[e], mv[e][i]);
          inc = add_rn(inc, mul_rn(wm, nr[e]));
          const float gwm = mul_rn(dinc, nr[e]);  // gradient of w_e msg_e
          s_n[e] += dinc * wm;
          s_w[e] += gwm * mv[e][i];
          E* dm = reinterpret_cast<E*>(g.dmsg[e].ptr) + (int64_t)b * g.dmsg[e].sb + (int64_t)t * g.dmsg[e].st +
                  (int64_t)h * g.dmsg[e].sh;
          dm[m] = from_f32<E>(mul_rn(gwm, wn[e]));
        }
      s_inc += d * inc;
      if (p.marginal) {
        const float lg = log1pf(cv[i]);
        s_log += d * lg;
        // out -= gexp log1p(counts): d counts = (-dout gexp) / (1 + counts)
        g.dcounts[row * M + m] = div_rn(-mul_rn(d, gexp), add_rn(1.f, cv[i]));
      }
    }
#pragma unroll
    for (int e = 0; e < GPA_ROUTE_MAX_INCOMING; ++e)
      if (e < NI) {
        const float sn = sum64(s_n[e]);
        if (lane == 0) g.dnorm[e][row] = sn;
      }
  }
  s_inc = sum64(s_inc);
  s_log = sum64(s_log);
#pragma unroll
  for (int e = 0; e < GPA_ROUTE_MAX_INCOMING; ++e) s_w[e] = sum64(s_w[e]);
  if (lane == 0) {
    part[wave][0] = s_inc;
    part[wave][1] = s_log;
#pragma unroll
    for (int e = 0; e < GPA_ROUTE_MAX_INCOMING; ++e) part[wave][2 + e] = s_w[e];
  }
  __syncthreads();
  if (threadIdx.x < 2 + NI) {
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < GPA_PRODUCT_ROWS; ++w) acc += part[w][threadIdx.x];
    g.partials[((int64_t)blockIdx.x * p.heads + h) * (2 + NI) + threadIdx.x] = acc;
  }
}

int check_product(const gpa_product_problem* p) {
  if (!p) return fail(GPA_HIP_EINVAL, "product read: null problem");
  if (p->batch < 1 || p->tokens < 1 || p->heads < 1) return fail(GPA_HIP_EINVAL, "product read: empty shape");
  if (p->slots < 1 || p->slots > GPA_ROUTE_MAX_WIDTH)
    return fail(GPA_HIP_EUNSUPPORTED, "product read: slots must be in [1, 256]");
  if (p->incoming < 1 || p->incoming > GPA_ROUTE_MAX_INCOMING)
    return fail(GPA_HIP_EUNSUPPORTED, "product read: 1 to 3 incoming edges");
  if (p->dtype != GPA_DTYPE_F32 && p->dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "product read: dtype");
  if (!p->base.ptr || !p->edge_weight || !p->gexp || (p->marginal && !p->counts.ptr))
    return fail(GPA_HIP_EINVAL, "product read: null operand");
  for (int e = 0; e < p->incoming; ++e)
    if (!p->msg[e].ptr || !p->norm[e].ptr) return fail(GPA_HIP_EINVAL, "product read: null message or norm");
  if ((int64_t)p->batch * p->tokens > 0x7fffffff - GPA_PRODUCT_ROWS)
    return fail(GPA_HIP_EUNSUPPORTED, "product read: too many rows");
  return GPA_HIP_OK;
}

dim3 product_grid(const gpa_product_problem& p) {
  return dim3((unsigned)(((int64_t)p.batch * p.tokens + GPA_PRODUCT_ROWS - 1) / GPA_PRODUCT_ROWS), (unsigned)p.heads);
}

}  // namespace
}  // namespace gpa

extern "C" int gpa_product_read_forward(const gpa_product_problem* problem, hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_product(problem)) return rc;
  if (!problem->out) return fail(GPA_HIP_EINVAL, "product read: null output");
  if (problem->dtype == GPA_DTYPE_BF16)
    hipLaunchKernelGGL(product_fwd<bf16_t>, product_grid(*problem), dim3(PNT), 0, stream, *problem);
  else
    hipLaunchKernelGGL(product_fwd<float>, product_grid(*problem), dim3(PNT), 0, stream, *problem);
  return check_launch("gpa_product_read_forward");
}

extern "C" int gpa_product_read_backward(const gpa_product_problem* problem, const gpa_product_grads* grads,
                                         hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_product(problem)) return rc;
  if (!grads || !grads->dout || !grads->partials || (problem->marginal && !grads->dcounts))
    return fail(GPA_HIP_EINVAL, "product read: null gradient buffer");
  for (int e = 0; e < problem->incoming; ++e)
    if (!grads->dmsg[e].ptr || !grads->dnorm[e]) return fail(GPA_HIP_EINVAL, "product read: null gradient buffer");
  if (problem->dtype == GPA_DTYPE_BF16)
    hipLaunchKernelGGL(product_bwd<bf16_t>, product_grid(*problem), dim3(PNT), 0, stream, *problem, *grads);
  else
    hipLaunchKernelGGL(product_bwd<float>, product_grid(*problem), dim3(PNT), 0, stream, *problem, *grads);
  return check_launch("gpa_product_read_backward");
}
