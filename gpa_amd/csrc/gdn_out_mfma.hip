// The read of the chunked GDN scan and the chunk-local part of its gradient
// on bf16 MFMA (gfx950 v_mfma_f32_32x32x16_bf16), one block per (chunk,
// stream), 4 waves.  Within a chunk of positions t, u:
//   P   = causal e^{G_t-G_u} Qn Kn^T
//   O   = diag(e^G) Qn S_n + P D                 (gdn_out_mfma)
//   dd0 = P^T dO,   o = diag(e^G) dO             (gdn_dd0_mfma, value-major)
// Qn and Kn are exact in bf16 (the model rounds them to the activation type);
// the fp32 operands S_n, D and P are split into bf16 hi + lo and multiplied as
// hi*hi + hi*lo + lo*hi, with fp32 accumulation.  Every global operand is read
// as 32 contiguous bytes per lane straight into MFMA fragments: Qn and Kn rows
// are position-major, and the chunk-start states and D are value-major, so a
// lane's eight contraction indices of one value column are contiguous.
// Reference: the output read of src/gpa/ops.py:29-46 in the chunked form.
#include <hip/hip_runtime.h>

#include "mfma_tiles.h"

namespace gpa {
namespace {

constexpr int OWAVES = 4, ONT = 64 * OWAVES;
constexpr int PLD = R + 8;  // bf16 pitch of 64-wide LDS rows (16-byte aligned rows)

__device__ __forceinline__ f32x16 mfma_bf16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Eight contiguous floats that are exact in bf16, as a fragment.
__device__ __forceinline__ bf16x8 frag_exact(const float* x) { return pack8(x); }

// Eight contiguous floats split into bf16 hi and lo = bf16(x - hi).
__device__ __forceinline__ void frag_split(const float* x, bf16x8& hi, bf16x8& lo) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(x), c = *reinterpret_cast<const f32x4*>(x + 4);
  const float v[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    hi[e] = (__bf16)v[e];
    lo[e] = (__bf16)(v[e] - (float)hi[e]);
  }
}

// The (rt, ct) 32x32 tile of P = causal e^{G_t-G_u} Qn Kn^T, with qa the Qn
// fragments of row tile rt (K16 k steps).  Lane l ends with column
// u = 32 ct + l%32 and rows t = 32 rt + acc_row(r, l/32).
template <int KM>
__device__ __forceinline__ f32x16 p_tile(const bf16x8 (&qa)[KM / 16], const float* kn, int K16, int K, int rt,
                                         int ct, int l, const float* gam_s) {
  const int li = l & 31, hh = l >> 5;
  f32x16 acc = {};
  const float* krow = kn + (32 * ct + li) * K + 8 * hh;
#pragma unroll
  for (int ks = 0; ks < KM / 16; ++ks)
    if (ks < K16) acc = mfma_bf16(qa[ks], frag_exact(krow + 16 * ks), acc);
  const int u = 32 * ct + li;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int t = 32 * rt + acc_row(r, hh);
    acc[r] = u <= t ? __expf(gam_s[t] - gam_s[u]) * acc[r] : 0.f;
  }
  return acc;
}

template <int KM>
__device__ __forceinline__ void load_q(bf16x8 (&qa)[KM / 16], const float* qn, int K16, int K, int rt, int l) {
  const float* qrow = qn + (32 * rt + (l & 31)) * K + 8 * (l >> 5);
#pragma unroll
  for (int ks = 0; ks < KM / 16; ++ks) qa[ks] = ks < K16 ? frag_exact(qrow + 16 * ks) : bf16x8{};
}

}  // namespace

// O = diag(e^G) Qn S_n + P D for one (chunk n, stream s); V <= 256.
template <int KM>
__global__ __launch_bounds__(ONT) void gdn_out_mfma(gpa_gdn_problem p, gpa_gdn_saved sv, gpa_operand out, int nch) {
  __shared__ __align__(16) __bf16 ph[R * PLD], pl[R * PLD];  // P hi / lo, [t][u]
  __shared__ float gam_s[R];
  const int n = blockIdx.x, s = blockIdx.y, b = s / p.heads, h = s % p.heads;
  const int K = p.kdim, V = p.vdim, K16 = K / 16, tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int li = l & 31, hh = l >> 5, rt = w & 1;
  if (tid < R) gam_s[tid] = sv.gam[rows_off(s, n, nch, 0, 1) + tid];
  bf16x8 qa[KM / 16];
  load_q<KM>(qa, sv.qn + rows_off(s, n, nch, 0, K), K16, K, rt, l);
  __syncthreads();
  {
    const f32x16 pt = p_tile<KM>(qa, sv.kn + rows_off(s, n, nch, 0, K), K16, K, rt, w >> 1, l, gam_s);
    const int u = 32 * (w >> 1) + li;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = 32 * rt + acc_row(r, hh);
      const __bf16 hi = (__bf16)pt[r];
      ph[t * PLD + u] = hi;
      pl[t * PLD + u] = (__bf16)(pt[r] - (float)hi);
    }
  }
  __syncthreads();
  const float* st = sv.states + state_off(s, n, nch, K, V);
  const float* dl = sv.delta + vc_off(s, n, nch, V);
  const int VT = (V + 31) / 32;
  for (int vt = w >> 1; vt < VT; vt += 2) {
    const int v = 32 * vt + li, vc = v < V ? v : V - 1;  // clamped column: loads stay in bounds
    f32x16 a1 = {}, a2 = {};
    const float* srow = st + (int64_t)vc * K + 8 * hh;
#pragma unroll
    for (int ks = 0; ks < KM / 16; ++ks)
      if (ks < K16) {
        bf16x8 bh, bl;
        frag_split(srow + 16 * ks, bh, bl);
        a1 = mfma_bf16(qa[ks], bh, a1);
        a2 = mfma_bf16(qa[ks], bl, a2);
      }
    f32x16 acc = a1 + a2;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] *= __expf(gam_s[32 * rt + acc_row(r, hh)]);
    const float* drow = dl + (int64_t)vc * R + 8 * hh;
#pragma unroll
    for (int us = 0; us < R / 16; ++us) {
      bf16x8 dh, dlo;
      frag_split(drow + 16 * us, dh, dlo);
      const int off = (32 * rt + li) * PLD + 16 * us + 8 * hh;
      const bf16x8 pa = *reinterpret_cast<const bf16x8*>(&ph[off]);
      const bf16x8 pb = *reinterpret_cast<const bf16x8*>(&pl[off]);
      acc = mfma_bf16(pa, dh, acc);
      acc = mfma_bf16(pa, dlo, acc);
      acc = mfma_bf16(pb, dh, acc);
    }
    if (v < V) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int tok = token_at(p, n, 32 * rt + acc_row(r, hh));
        if (tok >= 0)
          reinterpret_cast<bf16_t*>(out.ptr)[op_base(out, b, h) + (int64_t)tok * out.st + v] = f32_to_bf16(acc[r]);
      }
    }
  }
}

// dd0 = P^T dO and o = diag(e^G) dO (value-major [V][R]) for one (chunk n,
// stream s); V <= 256.
template <int KM>
__global__ __launch_bounds__(ONT) void gdn_dd0_mfma(gpa_gdn_problem p, gpa_gdn_saved sv, gpa_gdn_grads gr,
                                                     int nch) {
  __shared__ __align__(16) __bf16 ph[R * PLD], pl[R * PLD];  // P^T hi / lo, [u][t]
  __shared__ __align__(16) __bf16 dot[GPA_OUT_MFMA_MAX_V * PLD];  // dO^T, [v][t] (exact)
  __shared__ float gam_s[R];
  const int n = blockIdx.x, s = blockIdx.y, b = s / p.heads, h = s % p.heads;
  const int K = p.kdim, V = p.vdim, K16 = K / 16, tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int li = l & 31, hh = l >> 5, rt = w & 1;
  if (tid < R) gam_s[tid] = sv.gam[rows_off(s, n, nch, 0, 1) + tid];
  // dO rows into LDS, transposed: thread -> (row t, 8 consecutive values).
  const int V8 = (V + 7) / 8;
  for (int idx = tid; idx < R * V8; idx += ONT) {
    const int t = idx / V8, v0 = 8 * (idx - t * V8), tok = token_at(p, n, t);
    const bf16_t* src = reinterpret_cast<const bf16_t*>(gr.dout.ptr) + op_base(gr.dout, b, h) +
                        (int64_t)(tok >= 0 ? tok : 0) * gr.dout.st;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int v = v0 + e;
      const bf16_t x = (tok >= 0 && v < V) ? src[v] : bf16_t{0};
      if (v < V) reinterpret_cast<bf16_t*>(dot)[v * PLD + t] = x;
    }
  }
  bf16x8 qa[KM / 16];
  load_q<KM>(qa, sv.qn + rows_off(s, n, nch, 0, K), K16, K, rt, l);
  __syncthreads();
  {
    const f32x16 pt = p_tile<KM>(qa, sv.kn + rows_off(s, n, nch, 0, K), K16, K, rt, w >> 1, l, gam_s);
    const int u = 32 * (w >> 1) + li;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = 32 * rt + acc_row(r, hh);
      const __bf16 hi = (__bf16)pt[r];
      ph[u * PLD + t] = hi;
      pl[u * PLD + t] = (__bf16)(pt[r] - (float)hi);
    }
  }
  // o = diag(e^G) dO, value-major: thread -> (v, 4 consecutive rows).
  float* om = gr.o + vc_off(s, n, nch, V);
  for (int idx = tid; idx < V * (R / 4); idx += ONT) {
    const int v = idx / (R / 4), t0 = 4 * (idx - v * (R / 4));
    const bf16_t* x = reinterpret_cast<const bf16_t*>(dot) + v * PLD + t0;
    *reinterpret_cast<float4*>(om + (int64_t)v * R + t0) =
        make_float4(__expf(gam_s[t0]) * to_f32(x[0]), __expf(gam_s[t0 + 1]) * to_f32(x[1]),
                    __expf(gam_s[t0 + 2]) * to_f32(x[2]), __expf(gam_s[t0 + 3]) * to_f32(x[3]));
  }
  __syncthreads();
  float* d0 = gr.dd0 + vc_off(s, n, nch, V);
  const int VT = (V + 31) / 32, ut = rt;
  for (int vt = w >> 1; vt < VT; vt += 2) {
    const int v = 32 * vt + li, vc = v < V ? v : V - 1;
    f32x16 a1 = {}, a2 = {};
#pragma unroll
    for (int ts = 0; ts < R / 16; ++ts) {
      const int off = (32 * ut + li) * PLD + 16 * ts + 8 * hh;
      const bf16x8 pa = *reinterpret_cast<const bf16x8*>(&ph[off]);
      const bf16x8 pb = *reinterpret_cast<const bf16x8*>(&pl[off]);
      const bf16x8 bo = *reinterpret_cast<const bf16x8*>(&dot[vc * PLD + 16 * ts + 8 * hh]);
      a1 = mfma_bf16(pa, bo, a1);
      a2 = mfma_bf16(pb, bo, a2);
    }
    const f32x16 acc = a1 + a2;
    if (v < V) {
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4*>(d0 + (int64_t)v * R + 32 * ut + 8 * g + 4 * hh) =
            make_float4(acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]);
    }
  }
}

template <int KM>
int launch_out_mfma(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, gpa_operand out, int nch, hipStream_t st) {
  hipLaunchKernelGGL((gdn_out_mfma<KM>), dim3(nch, p.batch * p.heads), dim3(ONT), 0, st, p, sv, out, nch);
  return GPA_HIP_OK;
}

template <int KM>
int launch_dd0_mfma(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, const gpa_gdn_grads& gr, int nch,
                    hipStream_t st) {
  hipLaunchKernelGGL((gdn_dd0_mfma<KM>), dim3(nch, p.batch * p.heads), dim3(ONT), 0, st, p, sv, gr, nch);
  return GPA_HIP_OK;
}

template int launch_out_mfma<64>(const gpa_gdn_problem&, const gpa_gdn_saved&, gpa_operand, int, hipStream_t);
template int launch_out_mfma<128>(const gpa_gdn_problem&, const gpa_gdn_saved&, gpa_operand, int, hipStream_t);
template int launch_out_mfma<256>(const gpa_gdn_problem&, const gpa_gdn_saved&, gpa_operand, int, hipStream_t);
template int launch_dd0_mfma<64>(const gpa_gdn_problem&, const gpa_gdn_saved&, const gpa_gdn_grads&, int,
                                 hipStream_t);
template int launch_dd0_mfma<128>(const gpa_gdn_problem&, const gpa_gdn_saved&, const gpa_gdn_grads&, int,
                                  hipStream_t);
template int launch_dd0_mfma<256>(const gpa_gdn_problem&, const gpa_gdn_saved&, const gpa_gdn_grads&, int,
                                  hipStream_t);

}  // namespace gpa
