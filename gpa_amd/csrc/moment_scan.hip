// Gated moment scans: S_t = a_t o S_{t-1} + k_t v_t^T, y_t = S_t^T q_t per
// stream (reference src/gpa/ops.py:88-118 `linear_scan`, src/gpa/paper_dense.py
// :16-58 `moment_scan` and `decayed_counts`), and in reverse order the adjoint
// recursion of their backward.
//
// The recurrence is elementwise in S, so a state element never leaves the
// thread that holds it: one workgroup of 256 threads keeps one column block of
// one stream's float32 state in registers from the first token to the last.
// P adjacent lanes share a column, each holding RR consecutive rows, so the
// read y_t = S_t^T q_t is RR FMAs per lane and a P-lane shuffle sum.  The
// inputs of TC tokens are staged into LDS as float32 (decays as a = exp(g))
// one stage ahead through registers, with every load of a stage issued before
// any of them is used; a stage's outputs collect in LDS and leave in one
// coalesced pass.  Rows of a token are laid out per lane group with a stride
// of RR + 4 floats, so the P distinct 16-byte reads of an LDS instruction fall
// into distinct banks.
#include <hip/hip_runtime.h>

#include "gdn_common.h"

namespace gpa {
namespace {

constexpr int MT = 256;  // threads per workgroup

__device__ __forceinline__ int imin(int a, int b) { return a < b ? a : b; }

// Shape classes by key width: P lanes per column, RR rows per lane, TC tokens per stage.
template <int CLS> struct MClass;
template <> struct MClass<0> { static constexpr int P = 4, RR = 4, TC = 32; };    // K <= 16
template <> struct MClass<1> { static constexpr int P = 4, RR = 8, TC = 32; };    // K <= 32
template <> struct MClass<2> { static constexpr int P = 4, RR = 16, TC = 32; };   // K <= 64
template <> struct MClass<3> { static constexpr int P = 8, RR = 16, TC = 16; };   // K <= 128
template <> struct MClass<4> { static constexpr int P = 16, RR = 16, TC = 16; };  // K <= 256

__host__ __device__ inline int moment_class(int K) {
  return K <= 16 ? 0 : K <= 32 ? 1 : K <= 64 ? 2 : K <= 128 ? 3 : 4;
}
__host__ __device__ inline int moment_cols(int cls) { return MT / (cls <= 2 ? 4 : cls == 3 ? 8 : 16); }

template <int CLS>
struct MomentLds {
  static constexpr int P = MClass<CLS>::P, RR = MClass<CLS>::RR, TC = MClass<CLS>::TC;
  static constexpr int VC = MT / P, KLD = P * (RR + 4);
  float q[TC * KLD], k[TC * KLD];
  float ak[TC * KLD];  // per-row decays (GPA_GATE_KEY)
  float v[TC * VC], av[TC * VC], y[TC * VC];  // value columns, per-column decays, outputs
};

// Index of element d of a token row in the padded lane-group layout.
template <int RR>
__device__ __forceinline__ int row_slot(int d) {
  return (d / RR) * (RR + 4) + d % RR;
}

template <typename E, int CLS>
struct Stage {
  static constexpr int P = MClass<CLS>::P, RR = MClass<CLS>::RR, TC = MClass<CLS>::TC;
  static constexpr int VC = MT / P, KMAX = P * RR;
  static constexpr int NR = TC * KMAX / MT;  // row elements per thread per tensor
  static constexpr int NC = TC * VC / MT;    // column elements per thread
  static_assert(NR >= 1 && NC >= 1, "stage shape");
  float q[NR], k[NR], ak[NR];
  float v[NC], av[NC];
};

template <typename E, int CLS, bool GK>
__device__ __forceinline__ void stage_load(Stage<E, CLS>& st, const gpa_moment_problem& p, int b, int h, int c0,
                                           int t0) {
  using S = Stage<E, CLS>;
  const int tid = threadIdx.x;
  const int K = p.kdim, V = p.vdim, T = p.tokens;
  const E* qp = reinterpret_cast<const E*>(p.q.ptr) + op_base(p.q, b, h);
  const E* kp = reinterpret_cast<const E*>(p.k.ptr) + op_base(p.k, b, h);
  const E* vp = reinterpret_cast<const E*>(p.v.ptr) + op_base(p.v, b, h);
  const float* gp = p.gate != GPA_GATE_NONE ? reinterpret_cast<const float*>(p.g.ptr) + op_base(p.g, b, h) : nullptr;
  // Every load at a clamped (valid) address first; masks afterwards.
  E xq[S::NR], xk[S::NR], xv[S::NC];
  float xg[S::NR], xa[S::NC];
#pragma unroll
  for (int i = 0; i < S::NR; ++i) {
    const int e = tid + MT * i, t = imin(t0 + e / S::KMAX, T - 1), d = imin(e % S::KMAX, K - 1);
    xq[i] = qp[(int64_t)t * p.q.st + d];
    xk[i] = kp[(int64_t)t * p.k.st + d];
    if (GK) xg[i] = gp[(int64_t)t * p.g.st + d];
  }
#pragma unroll
  for (int i = 0; i < S::NC; ++i) {
    const int e = tid + MT * i, t = imin(t0 + e / S::VC, T - 1), c = imin(c0 + e % S::VC, V - 1);
    xv[i] = vp[(int64_t)t * p.v.st + c];
    if (!GK) {
      if (p.gate == GPA_GATE_TOKEN) xa[i] = gp[(int64_t)t * p.g.st];
      else if (p.gate == GPA_GATE_VALUE) xa[i] = gp[(int64_t)t * p.g.st + c];
      else xa[i] = 0.f;
    }
  }
#pragma unroll
  for (int i = 0; i < S::NR; ++i) {
    const int e = tid + MT * i;
    const bool ok = t0 + e / S::KMAX < T && e % S::KMAX < K;
    st.q[i] = ok ? to_f32(xq[i]) : 0.f;
    st.k[i] = ok ? to_f32(xk[i]) : 0.f;
    if (GK) st.ak[i] = ok ? __expf(xg[i]) : 1.f;
  }
#pragma unroll
  for (int i = 0; i < S::NC; ++i) {
    const int e = tid + MT * i;
    const bool ok = t0 + e / S::VC < T && c0 + e % S::VC < V;
    st.v[i] = ok ? to_f32(xv[i]) : 0.f;
    st.av[i] = (!GK && ok) ? __expf(xa[i]) : 1.f;
  }
}

template <typename E, int CLS, bool GK>
__device__ __forceinline__ void stage_store(const Stage<E, CLS>& st, MomentLds<CLS>& L) {
  using S = Stage<E, CLS>;
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < S::NR; ++i) {
    const int e = tid + MT * i, at = (e / S::KMAX) * MomentLds<CLS>::KLD + row_slot<S::RR>(e % S::KMAX);
    L.q[at] = st.q[i];
    L.k[at] = st.k[i];
    if (GK) L.ak[at] = st.ak[i];
  }
#pragma unroll
  for (int i = 0; i < S::NC; ++i) {
    const int e = tid + MT * i;
    L.v[e] = st.v[i];
    L.av[e] = st.av[i];
  }
}

// One problem's column block: blockIdx-relative workgroup `wg`.
template <typename E, int CLS, bool GK>
__device__ void moment_run(const gpa_moment_problem& p, int wg, MomentLds<CLS>& L) {
  constexpr int P = MClass<CLS>::P, RR = MClass<CLS>::RR, TC = MClass<CLS>::TC;
  constexpr int VC = MT / P, KLD = MomentLds<CLS>::KLD;
  const int tid = threadIdx.x, cl = tid / P, part = tid % P;
  const int nblk = (p.vdim + VC - 1) / VC;
  const int s = wg / nblk, c0 = (wg % nblk) * VC;
  const int b = s / p.heads, h = s % p.heads;
  const int K = p.kdim, V = p.vdim, T = p.tokens;
  const int col = c0 + cl, row0 = part * RR;
  const bool rev = p.reverse != 0;

  // State rows row0 .. row0 + RR - 1 of column `col` (zero past K and V).
  float S[RR];
  {
    const float* s0 = p.s0 ? p.s0 + (int64_t)b * p.s0_sb + (int64_t)h * p.s0_sh : nullptr;
    float x[RR];
#pragma unroll
    for (int r = 0; r < RR; ++r)
      x[r] = s0 ? s0[(int64_t)imin(row0 + r, K - 1) * V + imin(col, V - 1)] : 0.f;
#pragma unroll
    for (int r = 0; r < RR; ++r) S[r] = (row0 + r < K && col < V) ? x[r] : 0.f;
  }

  const int nst = (T + TC - 1) / TC;
  Stage<E, CLS> st;
  stage_load<E, CLS, GK>(st, p, b, h, c0, (rev ? nst - 1 : 0) * TC);
  E* yo = p.y_f32 ? nullptr : reinterpret_cast<E*>(p.y.ptr) + op_base(p.y, b, h);
  float* yf = p.y_f32 ? reinterpret_cast<float*>(p.y.ptr) + op_base(p.y, b, h) : nullptr;
  for (int si = 0; si < nst; ++si) {
    const int sn = rev ? nst - 1 - si : si, t0 = sn * TC;
    __syncthreads();  // the previous stage's LDS reads and output flush are done
    stage_store<E, CLS, GK>(st, L);
    if (si + 1 < nst) stage_load<E, CLS, GK>(st, p, b, h, c0, (rev ? sn - 1 : sn + 1) * TC);
    __syncthreads();
    for (int i = 0; i < TC; ++i) {
      const int tt = rev ? TC - 1 - i : i;
      const float* qr = &L.q[tt * KLD + part * (RR + 4)];
      const float* kr = &L.k[tt * KLD + part * (RR + 4)];
      float qv[RR], kv[RR], a[RR];
#pragma unroll
      for (int r = 0; r < RR; r += 4) {
        const float4 q4 = *reinterpret_cast<const float4*>(qr + r);
        const float4 k4 = *reinterpret_cast<const float4*>(kr + r);
        qv[r] = q4.x, qv[r + 1] = q4.y, qv[r + 2] = q4.z, qv[r + 3] = q4.w;
        kv[r] = k4.x, kv[r + 1] = k4.y, kv[r + 2] = k4.z, kv[r + 3] = k4.w;
        if (GK) {
          const float4 a4 = *reinterpret_cast<const float4*>(&L.ak[tt * KLD + part * (RR + 4) + r]);
          a[r] = a4.x, a[r + 1] = a4.y, a[r + 2] = a4.z, a[r + 3] = a4.w;
        }
      }
      const float vv = L.v[tt * VC + cl];
      if (!GK) {
        const float ac = L.av[tt * VC + cl];
#pragma unroll
        for (int r = 0; r < RR; ++r) a[r] = ac;
      }
      float part_sum = 0.f;
      if (!rev) {
#pragma unroll
        for (int r = 0; r < RR; ++r) S[r] = fmaf(a[r], S[r], kv[r] * vv);
#pragma unroll
        for (int r = 0; r < RR; ++r) part_sum = fmaf(qv[r], S[r], part_sum);
      } else {
#pragma unroll
        for (int r = 0; r < RR; ++r) S[r] = fmaf(kv[r], vv, S[r]);
#pragma unroll
        for (int r = 0; r < RR; ++r) part_sum = fmaf(qv[r], S[r], part_sum);
#pragma unroll
        for (int r = 0; r < RR; ++r) S[r] *= a[r];
      }
#pragma unroll
      for (int m = 1; m < P; m <<= 1) part_sum += __shfl_xor(part_sum, m, 64);
      if (part == 0) L.y[tt * VC + cl] = part_sum;
    }
    __syncthreads();
    constexpr int NC = TC * VC / MT;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int e = tid + MT * i, t = t0 + e / VC, c = c0 + e % VC;
      if (t < T && c < V) {
        const float y = L.y[e];
        if (yf) yf[(int64_t)t * p.y.st + c] = y;
        else yo[(int64_t)t * p.y.st + c] = from_f32<E>(y);
      }
    }
  }
  if (p.final && col < V) {
    float* f = p.final + ((int64_t)b * p.heads + h) * K * V;
#pragma unroll
    for (int r = 0; r < RR; ++r)
      if (row0 + r < K) f[(int64_t)(row0 + r) * V + col] = S[r];
  }
}

struct MomentPack {
  int n;
  int wg0[GPA_MOMENT_MAX_PACK];
  gpa_moment_problem p[GPA_MOMENT_MAX_PACK];
};

template <typename E, int CLS>
__device__ __forceinline__ void moment_dispatch_gate(const gpa_moment_problem& p, int wg, MomentLds<CLS>& L) {
  if (p.gate == GPA_GATE_KEY) moment_run<E, CLS, true>(p, wg, L);
  else moment_run<E, CLS, false>(p, wg, L);
}

// Workgroups wg0[i] .. wg0[i+1]-1 run problem i; the problem (and so its
// shape class and gate form) is uniform per workgroup.
template <typename E>
__global__ __launch_bounds__(MT) void moment_scan_pack(MomentPack pk) {
  typedef const __attribute__((address_space(4))) MomentPack* KernargPtr;
  const KernargPtr kp = (KernargPtr)__builtin_amdgcn_kernarg_segment_ptr();
  int pi = 0;
#pragma unroll 1
  for (int i = 1; i < kp->n; ++i)
    if ((int)blockIdx.x >= kp->wg0[i]) pi = i;
  gpa_moment_problem p;
  kernarg_copy(p, &kp->p[pi]);
  const int wg = (int)blockIdx.x - kp->wg0[pi];
  __shared__ union {
    MomentLds<0> c0;
    MomentLds<1> c1;
    MomentLds<2> c2;
    MomentLds<3> c3;
    MomentLds<4> c4;
  } lds;
  switch (moment_class(p.kdim)) {
    case 0: moment_dispatch_gate<E, 0>(p, wg, lds.c0); break;
    case 1: moment_dispatch_gate<E, 1>(p, wg, lds.c1); break;
    case 2: moment_dispatch_gate<E, 2>(p, wg, lds.c2); break;
    case 3: moment_dispatch_gate<E, 3>(p, wg, lds.c3); break;
    default: moment_dispatch_gate<E, 4>(p, wg, lds.c4); break;
  }
}

bool operand_ok(const gpa_operand& o) { return o.ptr != nullptr && o.sb >= 0 && o.st >= 0 && o.sh >= 0; }

int check_moment(const gpa_moment_problem* pp) {
  if (!pp) return fail(GPA_HIP_EINVAL, "moment scan: null problem");
  const gpa_moment_problem& p = *pp;
  if (p.batch < 1 || p.heads < 1 || p.tokens < 1)
    return fail(GPA_HIP_EINVAL, "moment scan: batch, heads and tokens must be positive");
  if (p.kdim < 1 || p.kdim > GPA_MOMENT_MAX_KDIM || p.vdim < 1)
    return fail(GPA_HIP_EINVAL, "moment scan: kdim must be 1..GPA_MOMENT_MAX_KDIM and vdim positive");
  if (p.dtype != GPA_DTYPE_F32 && p.dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "moment scan: dtype");
  if (p.gate < GPA_GATE_NONE || p.gate > GPA_GATE_VALUE) return fail(GPA_HIP_EINVAL, "moment scan: gate form");
  if (p.reverse != 0 && p.reverse != 1) return fail(GPA_HIP_EINVAL, "moment scan: reverse must be 0 or 1");
  if (!operand_ok(p.q) || !operand_ok(p.k) || !operand_ok(p.v) || !operand_ok(p.y))
    return fail(GPA_HIP_EINVAL, "moment scan: q, k, v and y are required (non-negative strides)");
  if (p.gate != GPA_GATE_NONE && !operand_ok(p.g)) return fail(GPA_HIP_EINVAL, "moment scan: gate operand required");
  if (p.s0 && (p.s0_sb < 0 || p.s0_sh < 0)) return fail(GPA_HIP_EINVAL, "moment scan: negative s0 stride");
  const int64_t streams = (int64_t)p.batch * p.heads;
  const int64_t wgs = streams * ((p.vdim + moment_cols(moment_class(p.kdim)) - 1) / moment_cols(moment_class(p.kdim)));
  if (wgs > INT32_MAX / 4) return fail(GPA_HIP_EINVAL, "moment scan: too many streams");
  return 0;
}

}  // namespace
}  // namespace gpa

extern "C" int gpa_moment_scan_many(const gpa_moment_problem* problems, int32_t n, hipStream_t stream) {
  using namespace gpa;
  if (!problems || n < 1 || n > GPA_MOMENT_MAX_PACK)
    return fail(GPA_HIP_EINVAL, "moment scan many: 1 to GPA_MOMENT_MAX_PACK problems");
  for (int i = 0; i < n; ++i) {
    if (int rc = check_moment(&problems[i])) return rc;
    if (problems[i].dtype != problems[0].dtype)
      return fail(GPA_HIP_EINVAL, "moment scan many: one element type per call");
  }
  MomentPack pk{};
  int64_t total = 0;
  for (int i = 0; i < n; ++i) {
    const gpa_moment_problem& p = problems[i];
    const int vc = moment_cols(moment_class(p.kdim));
    pk.p[i] = p;
    pk.wg0[i] = (int)total;
    total += (int64_t)p.batch * p.heads * ((p.vdim + vc - 1) / vc);
    if (total > INT32_MAX / 4) return fail(GPA_HIP_EINVAL, "moment scan many: too many workgroups");
  }
  pk.n = n;
  if (problems[0].dtype == GPA_DTYPE_BF16)
    hipLaunchKernelGGL((moment_scan_pack<bf16_t>), dim3((unsigned)total), dim3(MT), 0, stream, pk);
  else
    hipLaunchKernelGGL((moment_scan_pack<float>), dim3((unsigned)total), dim3(MT), 0, stream, pk);
  return check_launch("gpa_moment_scan_many");
}
