// Slot products and gate inputs of one level, fused over the key rows:
//   slot = k C^T                      (reference attention.py:176-177, einsum
//                                      "...hd,hmd->...hm" in the activation type)
//   raw  = unit(k) W_g                (attention.py:165; unit as ops.py:14-17)
// with C = center[level] [H][M][Dk] and W_g = gate_weight[level] [H][Dk][4],
// both rounded to the activation type.  Every product accumulates in float32
// and rounds its result to the activation type, as the reference's typed
// einsums do.  The gate nonlinearities on [B,T,H,4] stay with the caller.
//
// Backward: dk = round(round(dslot C) + round(normalize'(round(draw W_g^T)))),
// the two terms being the gradients the reference's autograd adds for the two
// uses of k; dW_g = round(sum_rows unit(k)^T draw); dC = round(sum_rows
// dslot^T k) runs as a row-reduction product (launch_tn_products).
//
// A workgroup owns 64 rows (two 32-row tiles) of one head; the key (forward)
// or dslot (backward) rows are read straight from global memory as MFMA A
// fragments, the weight rows as B fragments (C for the forward, C^T for the
// backward; both L2-resident per head).
#include <hip/hip_runtime.h>

#include "glue_rows.h"
#include "mfma_tiles.h"

namespace gpa {
namespace {

constexpr int SR = 64;  // rows per workgroup
constexpr int SNT = 256;

// Row offsets b*sb + t*st of the workgroup's rows r = row0 + i (rows past the
// end repeat the last one), computed once per workgroup.
__device__ __forceinline__ void row_table(int64_t* tab, const gpa_operand& o, int row0, int R, int T) {
  if (threadIdx.x < SR) {
    const int r = row0 + threadIdx.x < R ? row0 + threadIdx.x : R - 1, b = r / T, t = r - b * T;
    tab[threadIdx.x] = (int64_t)b * o.sb + (int64_t)t * o.st;
  }
}

__device__ __forceinline__ float wave_sum(float x) {
  x += __shfl_xor(x, 32);
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 8);
  x += __shfl_xor(x, 4);
  x += __shfl_xor(x, 2);
  return x + __shfl_xor(x, 1);
}

__device__ __forceinline__ bf16x8 ld_bf8(const bf16_t* p) {
  const uint4 w = *reinterpret_cast<const uint4*>(p);
  bf16x8 r;
  __builtin_memcpy(&r, &w, 16);
  return r;
}

// Forward.  Wave w: row tile w & 1; slot column tiles (w >> 1) + 2i.  Waves
// 0-1 also do the gate inputs of their row tile: lane l holds row l % 32,
// key columns 16 ks + 8 (l / 32) + 0..7 (its A fragments).
// ACT: the gate nonlinearities of each row follow in the same pass (inference,
// gpa_slot_gates_act_forward), from the gate inputs as rounded.
template <int KM, bool ACT>
__global__ __launch_bounds__(SNT) void slot_fwd(gpa_slot_problem p, gpa_gate_problem gp) {
  __shared__ int64_t key_off[SR], slot_off[SR], raw_off[SR];
  __shared__ float wg[KM * 4];
  const int h = blockIdx.y, row0 = blockIdx.x * SR, D = p.key_dim, M = p.slots, R = p.batch * p.tokens;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 31, hh = lane >> 5;
  const int K16 = D / 16, rt = wave & 1, ch = wave >> 1;
  if (tid < 64) {
    row_table(key_off, p.key, row0, R, p.tokens);
    row_table(slot_off, p.slot, row0, R, p.tokens);
    row_table(raw_off, p.raw, row0, R, p.tokens);
  }
  const bf16_t* gw = reinterpret_cast<const bf16_t*>(p.gate_w) + (int64_t)h * D * 4;
  for (int i = tid; i < D * 4; i += SNT) wg[i] = to_f32(gw[i]);
  __syncthreads();

  const int lrow = 32 * rt + li;
  const bf16_t* kp = reinterpret_cast<const bf16_t*>(p.key.ptr) + key_off[lrow] + (int64_t)h * p.key.sh + 8 * hh;
  bf16x8 a[KM / 16];
#pragma unroll
  for (int ks = 0; ks < KM / 16; ++ks) a[ks] = ld_bf8(kp + 16 * (ks < K16 ? ks : 0));
#pragma unroll
  for (int ks = 0; ks < KM / 16; ++ks)
    if (ks >= K16) a[ks] = bf16x8{};

  const bf16_t* cen = reinterpret_cast<const bf16_t*>(p.center) + (int64_t)h * M * D;
  bf16_t* slot = reinterpret_cast<bf16_t*>(p.slot.ptr) + (int64_t)h * p.slot.sh;
  // blockIdx.z splits the slot column tiles between workgroups (calls with few
  // rows, such as one-token decode); the gate inputs are done by z == 0.
  for (int ct = ch + 2 * (int)blockIdx.z; ct < M / 32; ct += 2 * (int)gridDim.z) {
    const bf16_t* cp = cen + (int64_t)(32 * ct + li) * D + 8 * hh;
    bf16x8 bfr[KM / 16];
#pragma unroll
    for (int ks = 0; ks < KM / 16; ++ks) bfr[ks] = ld_bf8(cp + 16 * (ks < K16 ? ks : 0));
    f32x16 acc = {};
#pragma unroll
    for (int ks = 0; ks < KM / 16; ++ks)
      if (ks < K16) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[ks], bfr[ks], acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 32 * rt + acc_row(r, hh);
      if (row0 + i < R) slot[slot_off[i] + 32 * ct + li] = from_f32<bf16_t>(acc[r]);
    }
  }

  if (ch == 0 && blockIdx.z == 0) {
    float ss = 0.f;
#pragma unroll
    for (int ks = 0; ks < KM / 16; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = (float)a[ks][e];
        ss += x * x;
      }
    ss += __shfl_xor(ss, 32);
    const float den = fmaxf(sqrtf(ss), 1e-6f);
    float g[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KM / 16; ++ks)
      if (ks < K16)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int d = 16 * ks + 8 * hh + e;
          const float u = round_as<bf16_t>((float)a[ks][e] / den);
#pragma unroll
          for (int c = 0; c < 4; ++c) g[c] += u * wg[4 * d + c];
        }
#pragma unroll
    for (int c = 0; c < 4; ++c) g[c] += __shfl_xor(g[c], 32);
    if (hh == 0 && row0 + lrow < R) {
      bf16_t* rp = reinterpret_cast<bf16_t*>(p.raw.ptr) + raw_off[lrow] + (int64_t)h * p.raw.sh;
#pragma unroll
      for (int c = 0; c < 4; ++c) rp[c] = from_f32<bf16_t>(g[c]);
      if (ACT) {
        float rr[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) rr[c] = round_as<bf16_t>(g[c]);
        gate_row(gp, h, (int64_t)(row0 + lrow) * p.heads + h, rr);
      }
    }
  }
}

// Backward.  Phase 1, 16 rows per wave, 64 lanes across the key columns: row
// norms, unit(k) . g (g = round(draw W_g^T)) and the dW_g partial sums.
// Phase 2: dk tiles on MFMA (wave w: row tile w & 1, key column tiles
// (w >> 1) + 2i), with the gate term added in the epilogue.
template <int KM>
__global__ __launch_bounds__(SNT) void slot_bwd(gpa_slot_problem p, gpa_slot_grads g) {
  __shared__ int64_t key_off[SR], ds_off[SR], dr_off[SR], dk_off[SR];
  __shared__ float wg[KM * 4], draw_s[SR][4], den_s[SR], dot_s[SR], red[4][KM * 4];
  const int h = blockIdx.y, row0 = blockIdx.x * SR, D = p.key_dim, M = p.slots, R = p.batch * p.tokens;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 31, hh = lane >> 5;
  if (tid < 64) {
    row_table(key_off, p.key, row0, R, p.tokens);
    row_table(ds_off, g.dslot, row0, R, p.tokens);
    row_table(dr_off, g.draw, row0, R, p.tokens);
    row_table(dk_off, g.dkey, row0, R, p.tokens);
  }
  const bf16_t* gw = reinterpret_cast<const bf16_t*>(p.gate_w) + (int64_t)h * D * 4;
  for (int i = tid; i < D * 4; i += SNT) wg[i] = to_f32(gw[i]);
  __syncthreads();

  // ---- phase 1
  constexpr int PD = KM / 64;  // key columns per lane
  const bf16_t* key = reinterpret_cast<const bf16_t*>(p.key.ptr) + (int64_t)h * p.key.sh;
  const bf16_t* draw = reinterpret_cast<const bf16_t*>(g.draw.ptr) + (int64_t)h * g.draw.sh;
  float wsum[PD][4] = {};
  {
    float xv[SR / 4][PD], dv[SR / 4][4];
#pragma unroll
    for (int j = 0; j < SR / 4; ++j) {  // loads first (clamped), then the row maths
      const int i = wave * (SR / 4) + j;
#pragma unroll
      for (int q = 0; q < PD; ++q) {
        const int d = lane + 64 * q;
        xv[j][q] = to_f32(key[key_off[i] + (d < D ? d : 0)]);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) dv[j][c] = to_f32(draw[dr_off[i] + c]);
    }
#pragma unroll
    for (int j = 0; j < SR / 4; ++j) {
      const int i = wave * (SR / 4) + j;
      const bool live = row0 + i < R;
      float ss = 0.f;
#pragma unroll
      for (int q = 0; q < PD; ++q) ss += lane + 64 * q < D ? xv[j][q] * xv[j][q] : 0.f;
      ss = wave_sum(ss);
      const float den = fmaxf(sqrtf(ss), 1e-6f);
      float dot = 0.f;
#pragma unroll
      for (int q = 0; q < PD; ++q) {
        const int d = lane + 64 * q;
        if (d < D) {
          float gu = 0.f;
#pragma unroll
          for (int c = 0; c < 4; ++c) gu += dv[j][c] * wg[4 * d + c];
          gu = round_as<bf16_t>(gu);
          const float uf = xv[j][q] / den;
          dot += uf * gu;
          const float ub = round_as<bf16_t>(uf);
#pragma unroll
          for (int c = 0; c < 4; ++c) wsum[q][c] += live ? ub * dv[j][c] : 0.f;
        }
      }
      dot = wave_sum(dot);
      if (lane == 0) {
        den_s[i] = (sqrtf(ss) > 1e-6f) ? den : -den;  // sign marks the clamped (eps) case
        dot_s[i] = dot;
      }
      if (lane == 0) {  // static indices: a lane-indexed register array would go to scratch
        draw_s[i][0] = dv[j][0];
        draw_s[i][1] = dv[j][1];
        draw_s[i][2] = dv[j][2];
        draw_s[i][3] = dv[j][3];
      }
    }
  }
#pragma unroll
  for (int q = 0; q < PD; ++q)
#pragma unroll
    for (int c = 0; c < 4; ++c) red[wave][4 * (lane + 64 * q) + c] = wsum[q][c];
  __syncthreads();
  for (int i = tid; i < D * 4; i += SNT)
    atomicAdd(&g.dgate_w[(int64_t)h * D * 4 + i], red[0][i] + red[1][i] + red[2][i] + red[3][i]);

  // ---- phase 2: dk = round(round(dslot C) + round(gate term))
  const int rt = wave & 1, ch = wave >> 1, M16 = M / 16;
  const int lrow = 32 * rt + li;
  const bf16_t* dsp =
      reinterpret_cast<const bf16_t*>(g.dslot.ptr) + ds_off[lrow] + (int64_t)h * g.dslot.sh + 8 * hh;
  const bf16_t* ct = reinterpret_cast<const bf16_t*>(p.center_t) + (int64_t)h * D * M;
  bf16_t* dk = reinterpret_cast<bf16_t*>(g.dkey.ptr) + (int64_t)h * g.dkey.sh;
  for (int dt = ch; dt < D / 32; dt += 2) {
    const int d = 32 * dt + li;
    const bf16_t* cp = ct + (int64_t)d * M + 8 * hh;
    f32x16 acc = {};
    // dslot row fragments (contraction m = 16 ms + 8 (l/32) + e, M <= 256) and
    // C^T fragments, 8 steps per group; the dslot rows are re-read per column
    // tile from L1/L2 rather than held across the loop
#pragma unroll
    for (int m0 = 0; m0 < 16; m0 += 8) {
      bf16x8 afr[8], bfr[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int ms = m0 + j < M16 ? m0 + j : 0;
        afr[j] = ld_bf8(dsp + 16 * ms);
        bfr[j] = ld_bf8(cp + 16 * ms);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (m0 + j < M16) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(afr[j], bfr[j], acc, 0, 0, 0);
    }
    float xk[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) xk[r] = to_f32(key[key_off[32 * rt + acc_row(r, hh)] + d]);
    float wd[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) wd[c] = wg[4 * d + c];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 32 * rt + acc_row(r, hh);
      if (row0 + i >= R) continue;
      float gu = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) gu += draw_s[i][c] * wd[c];
      gu = round_as<bf16_t>(gu);
      const float ds = den_s[i], den = fabsf(ds);
      const float dxg = round_as<bf16_t>(ds > 0.f ? (gu - (xk[r] / den) * dot_s[i]) / den : gu / den);
      dk[dk_off[i] + d] = from_f32<bf16_t>(round_as<bf16_t>(acc[r]) + dxg);
    }
  }
}

__global__ void slot_fill(float* x, int64_t n, bool round) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    x[i] = round ? round_as<bf16_t>(x[i]) : 0.f;
}

int check_slot(const gpa_slot_problem* p) {
  if (!p) return fail(GPA_HIP_EINVAL, "slot: null problem");
  if (p->dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "slot: bf16 activations only");
  if (p->batch < 1 || p->tokens < 1 || p->heads < 1) return fail(GPA_HIP_EINVAL, "slot: empty shape");
  if (p->key_dim < 16 || p->key_dim > 256 || p->key_dim % 16)
    return fail(GPA_HIP_EUNSUPPORTED, "slot: key width a multiple of 16 up to 256");
  if (p->slots < 32 || p->slots > 256 || p->slots % 32)
    return fail(GPA_HIP_EUNSUPPORTED, "slot: slots a multiple of 32 up to 256");
  if (!p->key.ptr || !p->center || !p->gate_w) return fail(GPA_HIP_EINVAL, "slot: null operand");
  if (p->key.st % 8 || p->key.sb % 8 || p->key.sh % 8 || (reinterpret_cast<uintptr_t>(p->key.ptr) & 15))
    return fail(GPA_HIP_EUNSUPPORTED, "slot: key rows must be 16-byte aligned");
  return GPA_HIP_OK;
}

}  // namespace
}  // namespace gpa

namespace gpa {
namespace {
int launch_slot_fwd(const gpa_slot_problem* problem, const gpa_gate_problem* gates, hipStream_t stream) {
  const int tiles = (problem->batch * problem->tokens + SR - 1) / SR;
  // Few row tiles (one-token decode): one workgroup per 64 slot columns.
  const int zsplit = tiles * problem->heads < 256 ? (problem->slots + 63) / 64 : 1;
  const dim3 grid(tiles, problem->heads, zsplit);
  const gpa_gate_problem none{};
  if (gates) {
    if (problem->key_dim <= 128)
      hipLaunchKernelGGL((slot_fwd<128, true>), grid, dim3(SNT), 0, stream, *problem, *gates);
    else
      hipLaunchKernelGGL((slot_fwd<256, true>), grid, dim3(SNT), 0, stream, *problem, *gates);
  } else {
    if (problem->key_dim <= 128)
      hipLaunchKernelGGL((slot_fwd<128, false>), grid, dim3(SNT), 0, stream, *problem, none);
    else
      hipLaunchKernelGGL((slot_fwd<256, false>), grid, dim3(SNT), 0, stream, *problem, none);
  }
  return GPA_HIP_OK;
}
}  // namespace
}  // namespace gpa

extern "C" int gpa_slot_gates_forward(const gpa_slot_problem* problem, hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_slot(problem)) return rc;
  if (!problem->slot.ptr || !problem->raw.ptr) return fail(GPA_HIP_EINVAL, "slot: null output");
  launch_slot_fwd(problem, nullptr, stream);
  return check_launch("gpa_slot_gates_forward");
}

extern "C" int gpa_slot_gates_act_forward(const gpa_slot_problem* problem, const gpa_gate_problem* gates,
                                          hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_slot(problem)) return rc;
  if (!problem->slot.ptr || !problem->raw.ptr) return fail(GPA_HIP_EINVAL, "slot: null output");
  if (!gates || !gates->bias || !gates->g_in || !gates->b_in || !gates->g_out || !gates->b_out)
    return fail(GPA_HIP_EINVAL, "slot: null gate output");
  if (gates->batch != problem->batch || gates->tokens != problem->tokens || gates->heads != problem->heads)
    return fail(GPA_HIP_EINVAL, "slot: the gate outputs must have the problem's batch, tokens and heads");
  launch_slot_fwd(problem, gates, stream);
  return check_launch("gpa_slot_gates_act_forward");
}

extern "C" int gpa_slot_gates_backward(const gpa_slot_problem* problem, const gpa_slot_grads* grads,
                                       hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_slot(problem)) return rc;
  if (!grads || !grads->dslot.ptr || !grads->draw.ptr || !grads->dkey.ptr || !grads->dcenter || !grads->dgate_w ||
      !problem->center_t)
    return fail(GPA_HIP_EINVAL, "slot: null gradient buffer");
  const gpa_slot_problem& p = *problem;
  if (grads->dslot.st % 8 || grads->dslot.sb % 8 || grads->dslot.sh % 8 ||
      (reinterpret_cast<uintptr_t>(grads->dslot.ptr) & 15))
    return fail(GPA_HIP_EUNSUPPORTED, "slot: dslot rows must be 16-byte aligned");
  const int R = p.batch * p.tokens, H = p.heads, D = p.key_dim, M = p.slots;
  // Rows r = b*T + t of the row-reduction operands must sit at r * (row stride).
  auto uniform = [&](const gpa_operand& o, int64_t& rs) {
    if (p.tokens == 1) rs = o.sb;
    else if (p.batch == 1 || o.sb == (int64_t)p.tokens * o.st) rs = o.st;
    else return false;
    return true;
  };
  int64_t rs_ds, rs_k;
  if (!uniform(grads->dslot, rs_ds) || !uniform(p.key, rs_k))
    return fail(GPA_HIP_EINVAL, "slot: dslot and key rows must be uniformly strided");
  const int64_t nw = (int64_t)H * D * 4;
  hipLaunchKernelGGL(slot_fill, dim3(16), dim3(256), 0, stream, grads->dgate_w, nw, false);
  const dim3 grid((R + SR - 1) / SR, H);
  if (D <= 128)
    hipLaunchKernelGGL(slot_bwd<128>, grid, dim3(SNT), 0, stream, p, *grads);
  else
    hipLaunchKernelGGL(slot_bwd<256>, grid, dim3(SNT), 0, stream, p, *grads);
  hipLaunchKernelGGL(slot_fill, dim3(16), dim3(256), 0, stream, grads->dgate_w, nw, true);
  const TnProduct dc{grads->dslot.ptr, rs_ds, grads->dslot.sh, M, p.key.ptr, rs_k, p.key.sh, D, grads->dcenter};
  if (int rc = launch_tn_products(&dc, 1, H, R, true, stream)) return rc;
  return check_launch("gpa_slot_gates_backward");
}
