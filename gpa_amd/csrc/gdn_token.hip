// One-token GDN step of a group of streams without saved intermediates (the
// inference decode of the chunk model at T = 1): reference src/gpa/ops.py:29-42
// (gdn_update) then :45-46 (memory_read) for every stream of the group.
//
// HBM bound: each stream's fp32 state is read once and written once.  A
// workgroup holds one column block of one stream's state in registers (64
// columns, thread t: columns 4 (t % 16) .. +3 of rows t / 16 + 16 i; 32
// columns for K > 128), so the prediction u(k)^T (a S), the update and the
// read u(q)^T S' all come from the one load.
#include "token_step.h"

namespace gpa {
namespace {

template <typename E, int NI>
__global__ __launch_bounds__(SNT) void gdn_token_step(gpa_gdn_problem p, float* fin, gpa_operand out) {
  __shared__ TokenLds<NI> lds;
  token_run<E, NI>(p, fin, out, blockIdx.x, threadIdx.x, lds, gpa_token_slot{});
}

// Several problems with the same element type in one launch: workgroups
// wg0[i] .. wg0[i+1]-1 run problem i, in its row class ni[i] (4, 8 or 16).
struct TokenPack {
  int n;
  int wg0[GPA_TOKEN_MAX_PACK];
  int ni[GPA_TOKEN_MAX_PACK];
  float* fin[GPA_TOKEN_MAX_PACK];
  gpa_operand out[GPA_TOKEN_MAX_PACK];
  gpa_gdn_problem p[GPA_TOKEN_MAX_PACK];
};

// The pack is the kernel's only argument: its entries are read through the
// kernel-argument pointer with a uniform index, as scalar loads (indexing the
// by-value argument would copy it to scratch).  The row classes share one
// launch (a workgroup's class is uniform), so the relation edges or the
// outer memories of every key width end in one kernel, not one per class.
template <typename E>
__global__ __launch_bounds__(SNT) void gdn_token_step_pack(TokenPack pk) {
  typedef const __attribute__((address_space(4))) TokenPack* KernargPtr;
  const KernargPtr kp = (KernargPtr)__builtin_amdgcn_kernarg_segment_ptr();
  int pi = 0;
#pragma unroll 1
  for (int i = 1; i < kp->n; ++i)
    if ((int)blockIdx.x >= kp->wg0[i]) pi = i;
  gpa_gdn_problem p;
  gpa_operand out;
  kernarg_copy(p, &kp->p[pi]);
  kernarg_copy(out, &kp->out[pi]);
  __shared__ union {
    TokenLds<4> c4;
    TokenLds<8> c8;
    TokenLds<16> c16;
  } lds;
  const int wg = (int)blockIdx.x - kp->wg0[pi], ni = kp->ni[pi];
  const gpa_token_slot none{};
  if (ni == 4) token_run<E, 4>(p, kp->fin[pi], out, wg, threadIdx.x, lds.c4, none);
  else if (ni == 8) token_run<E, 8>(p, kp->fin[pi], out, wg, threadIdx.x, lds.c8, none);
  else token_run<E, 16>(p, kp->fin[pi], out, wg, threadIdx.x, lds.c16, none);
}

template <typename E>
void launch_token(const gpa_gdn_problem& p, float* fin, gpa_operand out, hipStream_t stream) {
  const dim3 grid((unsigned)token_workgroups(p));
  switch (token_rows(p)) {
    case 4: hipLaunchKernelGGL((gdn_token_step<E, 4>), grid, dim3(SNT), 0, stream, p, fin, out); break;
    case 8: hipLaunchKernelGGL((gdn_token_step<E, 8>), grid, dim3(SNT), 0, stream, p, fin, out); break;
    default: hipLaunchKernelGGL((gdn_token_step<E, 16>), grid, dim3(SNT), 0, stream, p, fin, out);
  }
}


}  // namespace
}  // namespace gpa

extern "C" int gpa_gdn_token_step(const gpa_gdn_problem* problem, float* final_state, gpa_operand out,
                                  hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_token(problem, final_state, out)) return rc;
  const gpa_gdn_problem& p = *problem;
  if (p.dtype == GPA_DTYPE_BF16) launch_token<bf16_t>(p, final_state, out, stream);
  else launch_token<float>(p, final_state, out, stream);
  return check_launch("gpa_gdn_token_step");
}

extern "C" int gpa_gdn_token_step_many(const gpa_gdn_problem* problems, float* const* final_states,
                                       const gpa_operand* outs, int32_t n, hipStream_t stream) {
  using namespace gpa;
  if (!problems || !final_states || !outs || n < 1 || n > GPA_TOKEN_MAX_PACK)
    return fail(GPA_HIP_EINVAL, "token step many: 1 to GPA_TOKEN_MAX_PACK problems with finals and outs");
  for (int i = 0; i < n; ++i)
    if (int rc = check_token(&problems[i], final_states[i], outs[i])) return rc;
  // One launch per element type present, problems in call order.
  for (int dt = 0; dt < 2; ++dt) {
    TokenPack pk{};
    int64_t total = 0;
    for (int i = 0; i < n; ++i) {
      const gpa_gdn_problem& p = problems[i];
      if (p.dtype != (dt ? GPA_DTYPE_BF16 : GPA_DTYPE_F32)) continue;
      pk.p[pk.n] = p;
      pk.fin[pk.n] = final_states[i];
      pk.out[pk.n] = outs[i];
      pk.ni[pk.n] = token_rows(p);
      pk.wg0[pk.n] = (int)total;
      total += token_workgroups(p);
      if (total > INT32_MAX / 2) return fail(GPA_HIP_EINVAL, "token step many: too many workgroups");
      ++pk.n;
    }
    if (!pk.n) continue;
    if (dt) hipLaunchKernelGGL((gdn_token_step_pack<bf16_t>), dim3((unsigned)total), dim3(SNT), 0, stream, pk);
    else hipLaunchKernelGGL((gdn_token_step_pack<float>), dim3((unsigned)total), dim3(SNT), 0, stream, pk);
  }
  return check_launch("gpa_gdn_token_step_many");
}
