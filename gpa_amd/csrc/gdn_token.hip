// One-token GDN step of a group of streams without saved intermediates (the
// inference decode of the chunk model at T = 1): reference src/gpa/ops.py:29-42
// (gdn_update) then :45-46 (memory_read) for every stream of the group.
//
// HBM bound: each stream's fp32 state is read once and written once.  A
// workgroup holds one 64-column block of one stream's state in registers
// (thread t: columns 4 (t % 16) .. +3 of rows t / 16 + 16 i), so the
// prediction u(k)^T (a S), the update and the read u(q)^T S' all come from the
// one load.
#include "token_step.h"

namespace gpa {
namespace {

template <typename E, int NI>
__global__ __launch_bounds__(SNT) void gdn_token_step(gpa_gdn_problem p, float* fin, gpa_operand out) {
  __shared__ TokenLds<NI> lds;
  token_run<E, NI>(p, fin, out, blockIdx.x, threadIdx.x, lds);
}

// Several problems with the same element type and row class in one launch:
// workgroups wg0[i] .. wg0[i+1]-1 run problem i.
struct TokenPack {
  int n;
  int wg0[GPA_TOKEN_MAX_PACK];
  float* fin[GPA_TOKEN_MAX_PACK];
  gpa_operand out[GPA_TOKEN_MAX_PACK];
  gpa_gdn_problem p[GPA_TOKEN_MAX_PACK];
};

// The pack is the kernel's only argument: its entries are read through the
// kernel-argument pointer with a uniform index, as scalar loads (indexing the
// by-value argument would copy it to scratch).
template <typename E, int NI>
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
  __shared__ TokenLds<NI> lds;
  token_run<E, NI>(p, kp->fin[pi], out, (int)blockIdx.x - kp->wg0[pi], threadIdx.x, lds);
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

template <typename E>
void launch_token_pack(const TokenPack& pk, int rows, unsigned grid, hipStream_t stream) {
  switch (rows) {
    case 4: hipLaunchKernelGGL((gdn_token_step_pack<E, 4>), dim3(grid), dim3(SNT), 0, stream, pk); break;
    case 8: hipLaunchKernelGGL((gdn_token_step_pack<E, 8>), dim3(grid), dim3(SNT), 0, stream, pk); break;
    default: hipLaunchKernelGGL((gdn_token_step_pack<E, 16>), dim3(grid), dim3(SNT), 0, stream, pk);
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
  // One launch per (element type, row class) present, problems in call order.
  for (int dt = 0; dt < 2; ++dt)
    for (int rows = 4; rows <= 16; rows *= 2) {
      TokenPack pk{};
      int64_t total = 0;
      for (int i = 0; i < n; ++i) {
        const gpa_gdn_problem& p = problems[i];
        if (p.dtype != (dt ? GPA_DTYPE_BF16 : GPA_DTYPE_F32) || token_rows(p) != rows) continue;
        pk.p[pk.n] = p;
        pk.fin[pk.n] = final_states[i];
        pk.out[pk.n] = outs[i];
        pk.wg0[pk.n] = (int)total;
        total += token_workgroups(p);
        ++pk.n;
      }
      if (!pk.n) continue;
      if (total > INT32_MAX / 2) return fail(GPA_HIP_EINVAL, "token step many: too many workgroups");
      if (dt) launch_token_pack<bf16_t>(pk, rows, (unsigned)total, stream);
      else launch_token_pack<float>(pk, rows, (unsigned)total, stream);
    }
  return check_launch("gpa_gdn_token_step_many");
}
