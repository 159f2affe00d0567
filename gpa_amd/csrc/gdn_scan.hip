// Chunked gated-delta-rule (GDN) scan for gfx950: forward and backward.
//
// Per stream, S_t = e^{g_t} (I - b_t k_t k_t^T) S_{t-1} + b_t k_t v_t^T and
// o_t = q_t^T S_t with k, q L2-normalised (reference src/gpa/ops.py:29-46,
// 80-85).  Within a chunk of positions with in-chunk cumulative log decay G:
//   A_ts = b_t e^{G_t-G_s} k_t.k_s (s<t),  T = (I+A)^-1,
//   U = T diag(b) V,  W = T diag(b e^G) K,  D = U - W S_n,
//   O = diag(e^G) Q S_n + (causal e^{G_t-G_s} Q K^T) D,
//   S_{n+1} = e^{G_C} S_n + (diag(e^{G_C-G}) K)^T D.
// Kernels:
//   gdn_prep_mfma  chunk-parallel: normalise, G, T, W, U (gdn_prep_mfma.hip)
//   gdn_state_fwd  sequential over chunks, parallel over (stream, 32-column tile):
//                  S_n (saved), D
//   gdn_out_fwd    chunk-parallel: O
//   gdn_dd0        chunk-parallel: P^T dO (the in-chunk part of dD)
//   gdn_state_bwd  reverse sequential: dS at every chunk end, dD
//   gdn_chunk_bwd  chunk-parallel: dq, dk, dv, dg, dbeta
// All intermediates are float32; q/k/v/out may be bf16 (rounded exactly where
// the reference rounds: the normalised keys/queries and the read).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <stdio.h>
#include <type_traits>

#include "gpa_hip.h"
#include "gpa_common.h"
#include "gdn_common.h"
#include "gdn_strip.h"

namespace gpa {

// ---------------------------------------------------------------------------
// gdn_state_fwd: block (column tile blockIdx.x, stream blockIdx.y), loops chunks.
template <int KM>
__global__ __launch_bounds__(NT) void gdn_state_fwd(gpa_gdn_problem p, gpa_gdn_saved sv, int nch) {
  extern __shared__ float smem[];
  float* st_s = smem;                   // [KM][VT+1]
  float* w_s = st_s + KM * (VT + 1);    // [R][LDS_]
  float* d_s = w_s + R * LDS_;          // [R][VT+1]
  float* gam_s = d_s + R * (VT + 1);    // [R]
  float* rs_s = gam_s + R;              // [R] row scales
  const int s = blockIdx.y, b = s / p.heads, h = s % p.heads;
  const int K = p.kdim, V = p.vdim, tid = threadIdx.x;
  const int r = tid / VT, c = tid % VT;  // r in 0..7
  const int v = blockIdx.x * VT + c;
  const bool vok = v < V;

  for (int i = 0; i < KM / 8; ++i) {
    const int k = r + 8 * i;
    st_s[k * (VT + 1) + c] = (p.s0 && k < K && vok)
        ? p.s0[(int64_t)b * p.s0_sb + (int64_t)h * p.s0_sh + (int64_t)k * V + v] : 0.f;
  }
  __syncthreads();
  for (int n = 0; n < nch; ++n) {
    const int64_t so = state_off(s, n, nch, K, V);
    if (vok)
      for (int i = 0; i < KM / 8; ++i) {
        const int k = r + 8 * i;
        if (k < K) sv.states[so + (int64_t)v * K + k] = st_s[k * (VT + 1) + c];
      }
    // D = U - W S
    const float* um = sv.u + vc_off(s, n, nch, V);
    float acc[R / 8];
#pragma unroll
    for (int j = 0; j < R / 8; ++j) acc[j] = vok ? um[(int64_t)v * R + r + 8 * j] : 0.f;
    for (int k0 = 0; k0 < KM; k0 += KS) {
      __syncthreads();
      stage_rows(w_s, sv.w + rows_off(s, n, nch, 0, K), K, k0, nullptr);
      __syncthreads();
      for (int kk = 0; kk < KS; ++kk) {
        const float sk = st_s[(k0 + kk) * (VT + 1) + c];
#pragma unroll
        for (int j = 0; j < R / 8; ++j) acc[j] -= w_s[(r + 8 * j) * LDS_ + kk] * sk;
      }
    }
    float* dm = sv.delta + vc_off(s, n, nch, V);
#pragma unroll
    for (int j = 0; j < R / 8; ++j) {
      d_s[(r + 8 * j) * (VT + 1) + c] = acc[j];
      if (vok) dm[(int64_t)v * R + r + 8 * j] = acc[j];
    }
    if (tid < R) gam_s[tid] = sv.gam[rows_off(s, n, nch, 0, 1) + tid];
    __syncthreads();
    const float gc = gam_s[R - 1];
    const float decay = __expf(gc);
    if (tid < R) rs_s[tid] = __expf(gc - gam_s[tid]);
    // S = e^{G_C} S + (diag(e^{G_C-G}) Kn)^T D
    for (int k0 = 0; k0 < KM; k0 += KS) {
      __syncthreads();
      stage_rows(w_s, sv.kn + rows_off(s, n, nch, 0, K), K, k0, rs_s);
      __syncthreads();
#pragma unroll
      for (int i = 0; i < KS / 8; ++i) {
        const int kk = r + 8 * i;
        float x = decay * st_s[(k0 + kk) * (VT + 1) + c];
        for (int t = 0; t < R; ++t) x += w_s[t * LDS_ + kk] * d_s[t * (VT + 1) + c];
        st_s[(k0 + kk) * (VT + 1) + c] = x;
      }
    }
    __syncthreads();
  }
  if (vok)
    for (int i = 0; i < KM / 8; ++i) {
      const int k = r + 8 * i;
      if (k < K) sv.final[(int64_t)s * K * V + (int64_t)k * V + v] = st_s[k * (VT + 1) + c];
    }
}

// P = causal e^{G_t-G_s} Qn Kn^T into p_s ([R][LDR]); uses two R x KS slices.
template <int KM>
__device__ void build_p(float* p_s, float* a_s, float* b_s, const float* qn, const float* kn,
                        const float* gam_s, int K) {
  const int tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < KM; k0 += KS) {
    __syncthreads();
    stage_rows(a_s, qn, K, k0, nullptr);
    stage_rows(b_s, kn, K, k0, nullptr);
    __syncthreads();
    for (int kk = 0; kk < KS; ++kk) {
      float a[4], c[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = a_s[(4 * ty + i) * LDS_ + kk];
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = b_s[(tx + 16 * j) * LDS_ + kk];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * c[j];
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 4 * ty + i, u = tx + 16 * j;
      p_s[t * LDR + u] = (u <= t) ? __expf(gam_s[t] - gam_s[u]) * acc[i][j] : 0.f;
    }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// gdn_out_fwd: O = diag(e^G) Qn S_n + P D, one block per (chunk, stream).
template <typename E, int KM>
__global__ __launch_bounds__(NT) void gdn_out_fwd(gpa_gdn_problem p, gpa_gdn_saved sv, gpa_operand out,
                                                   int nch) {
  extern __shared__ float smem[];
  float* p_s = smem;              // [R][LDR]
  float* a_s = p_s + R * LDR;     // [R][LDS_]
  float* b_s = a_s + R * LDS_;    // [R][LDS_]  (also KS x 64 state slice)
  float* gam_s = b_s + R * LDS_;  // [R]
  const int n = blockIdx.x, s = blockIdx.y, b = s / p.heads, h = s % p.heads;
  const int K = p.kdim, V = p.vdim, tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
  if (tid < R) gam_s[tid] = sv.gam[rows_off(s, n, nch, 0, 1) + tid];
  __syncthreads();
  const float* qn = sv.qn + rows_off(s, n, nch, 0, K);
  build_p<KM>(p_s, a_s, b_s, qn, sv.kn + rows_off(s, n, nch, 0, K), gam_s, K);
  const float* st = sv.states + state_off(s, n, nch, K, V);
  const float* dl = sv.delta + vc_off(s, n, nch, V);
  for (int v0 = 0; v0 < V; v0 += 64) {
    float acc[4][4] = {};
    for (int k0 = 0; k0 < KM; k0 += KS) {
      __syncthreads();
      stage_rows(a_s, qn, K, k0, nullptr);
      for (int idx = tid; idx < KS * 64; idx += NT) {
        const int kk = idx % KS, c = idx / KS;
        b_s[kk * LDS_ + c] = (k0 + kk < K && v0 + c < V) ? st[(int64_t)(v0 + c) * K + k0 + kk] : 0.f;
      }
      __syncthreads();
      for (int kk = 0; kk < KS; ++kk) {
        float a[4], c[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = a_s[(4 * ty + i) * LDS_ + kk];
#pragma unroll
        for (int j = 0; j < 4; ++j) c[j] = b_s[kk * LDS_ + tx + 16 * j];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * c[j];
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float e = __expf(gam_s[4 * ty + i]);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] *= e;
    }
    __syncthreads();
    for (int idx = tid; idx < R * 64; idx += NT) {
      const int u = idx % R, c = idx / R;
      b_s[u * LDS_ + c] = v0 + c < V ? dl[(int64_t)(v0 + c) * R + u] : 0.f;
    }
    __syncthreads();
    for (int u = 0; u < R; ++u) {
      float a[4], c[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = p_s[(4 * ty + i) * LDR + u];
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = b_s[u * LDS_ + tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * c[j];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = token_at(p, n, 4 * ty + i);
      if (t < 0) continue;
      E* o = reinterpret_cast<E*>(out.ptr) + op_base(out, b, h) + (int64_t)t * out.st;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int v = v0 + tx + 16 * j;
        if (v < V) o[v] = from_f32<E>(acc[i][j]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// gdn_dd0: dd0 = P^T dO (the part of dD not carried by the state), and
// o = diag(e^G) dO, both value-major [V][R] per chunk.
template <typename E, int KM>
__global__ __launch_bounds__(NT) void gdn_dd0(gpa_gdn_problem p, gpa_gdn_saved sv, gpa_gdn_grads gr,
                                               int nch) {
  extern __shared__ float smem[];
  float* p_s = smem;
  float* a_s = p_s + R * LDR;
  float* b_s = a_s + R * LDS_;
  float* gam_s = b_s + R * LDS_;
  const int n = blockIdx.x, s = blockIdx.y, b = s / p.heads, h = s % p.heads;
  const int K = p.kdim, V = p.vdim, tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
  if (tid < R) gam_s[tid] = sv.gam[rows_off(s, n, nch, 0, 1) + tid];
  __syncthreads();
  build_p<KM>(p_s, a_s, b_s, sv.qn + rows_off(s, n, nch, 0, K), sv.kn + rows_off(s, n, nch, 0, K), gam_s, K);
  // dd0 and o are value-major for the FMA state kernels and in fragment order
  // (ufrag_idx) for the MFMA ones (bf16, K a multiple of 16).
  const bool frag = std::is_same<E, bf16_t>::value && K % 16 == 0;
  float* d0 = gr.dd0 + (frag ? ufrag_off(s, n, nch, V) : vc_off(s, n, nch, V));
  float* om = gr.o + (frag ? ufrag_off(s, n, nch, V) : vc_off(s, n, nch, V));
  auto at = [&](int v, int r) -> int64_t { return frag ? ufrag_elem(v, r) : (int64_t)v * R + r; };
  for (int v0 = 0; v0 < V; v0 += 64) {
    __syncthreads();
    for (int idx = tid; idx < R * 64; idx += NT) {
      const int r = idx / 64, c = idx % 64;
      const int t = token_at(p, n, r);
      b_s[r * LDS_ + c] = (t >= 0 && v0 + c < V) ? op_load<E>(gr.dout, b, h, t, v0 + c) : 0.f;
    }
    __syncthreads();
    for (int idx = tid; idx < R * 64; idx += NT) {
      const int r = idx % R, c = idx / R;
      if (v0 + c < V) om[at(v0 + c, r)] = __expf(gam_s[r]) * b_s[r * LDS_ + c];
      else if (frag && v0 + c < ufrag_v(V)) om[at(v0 + c, r)] = 0.f;
    }
    float acc[4][4] = {};
    for (int u = 0; u < R; ++u) {  // acc[t'][v] += P[u][t'] dO[u][v]
      float a[4], c[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = p_s[u * LDR + 4 * ty + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = b_s[u * LDS_ + tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * c[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int v = v0 + tx + 16 * j;  // four consecutive rows are contiguous in both layouts
      if (v < V)
        *reinterpret_cast<float4*>(&d0[at(v, 4 * ty)]) = make_float4(acc[0][j], acc[1][j], acc[2][j], acc[3][j]);
      else if (frag && v < ufrag_v(V))
        *reinterpret_cast<float4*>(&d0[at(v, 4 * ty)]) = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
}

// ---------------------------------------------------------------------------
// gdn_state_bwd: reverse sequential dS; writes dS at every chunk end and dD.
template <typename E, int KM>
__global__ __launch_bounds__(NT) void gdn_state_bwd(gpa_gdn_problem p, gpa_gdn_saved sv, gpa_gdn_grads gr,
                                                     int nch) {
  extern __shared__ float smem[];
  float* ds_s = smem;                   // [KM][VT+1]
  float* x_s = ds_s + KM * (VT + 1);    // [R][LDS_]
  float* y_s = x_s + R * LDS_;          // [R][LDS_]
  float* dd_s = y_s + R * LDS_;         // [R][VT+1]
  float* o_s = dd_s + R * (VT + 1);     // [R][VT+1]
  float* gam_s = o_s + R * (VT + 1);    // [R]
  float* rs_s = gam_s + R;              // [R]
  const int s = blockIdx.y, b = s / p.heads, h = s % p.heads;
  const int K = p.kdim, V = p.vdim, tid = threadIdx.x;
  const int r = tid / VT, c = tid % VT;
  const int v = blockIdx.x * VT + c;
  const bool vok = v < V;
  const bool has_q = p.q.ptr != nullptr && gr.dout.ptr != nullptr;

  for (int i = 0; i < KM / 8; ++i) {
    const int k = r + 8 * i;
    ds_s[k * (VT + 1) + c] = (gr.dfinal && k < K && vok) ? gr.dfinal[(int64_t)s * K * V + (int64_t)k * V + v] : 0.f;
  }
  for (int n = nch - 1; n >= 0; --n) {
    __syncthreads();
    const int64_t so = state_off(s, n, nch, K, V);
    if (vok)
      for (int i = 0; i < KM / 8; ++i) {
        const int k = r + 8 * i;
        if (k < K) gr.dhend[so + (int64_t)v * K + k] = ds_s[k * (VT + 1) + c];
      }
    if (tid < R) gam_s[tid] = sv.gam[rows_off(s, n, nch, 0, 1) + tid];
    __syncthreads();
    const float gc = gam_s[R - 1];
    if (tid < R) rs_s[tid] = __expf(gc - gam_s[tid]);
    // dD = dd0 + diag(e^{G_C-G}) Kn dS
    const float* d0 = gr.dd0 ? gr.dd0 + vc_off(s, n, nch, V) : nullptr;
    const float* om = has_q ? gr.o + vc_off(s, n, nch, V) : nullptr;
    float* ddm = gr.ddelta + vc_off(s, n, nch, V);
    float acc[R / 8];
#pragma unroll
    for (int j = 0; j < R / 8; ++j) acc[j] = (d0 && vok) ? d0[(int64_t)v * R + r + 8 * j] : 0.f;
    for (int k0 = 0; k0 < KM; k0 += KS) {
      __syncthreads();
      stage_rows(x_s, sv.kn + rows_off(s, n, nch, 0, K), K, k0, rs_s);
      __syncthreads();
      for (int kk = 0; kk < KS; ++kk) {
        const float d = ds_s[(k0 + kk) * (VT + 1) + c];
#pragma unroll
        for (int j = 0; j < R / 8; ++j) acc[j] += x_s[(r + 8 * j) * LDS_ + kk] * d;
      }
    }
#pragma unroll
    for (int j = 0; j < R / 8; ++j) {
      const int t = r + 8 * j;
      dd_s[t * (VT + 1) + c] = acc[j];
      if (vok) ddm[(int64_t)v * R + t] = acc[j];
      o_s[t * (VT + 1) + c] = (om && vok) ? om[(int64_t)v * R + t] : 0.f;
    }
    // dS_prev = e^{G_C} dS + Qn^T diag(e^G) dO - W^T dD + dstates[n]
    const float decay = __expf(gc);
    for (int k0 = 0; k0 < KM; k0 += KS) {
      __syncthreads();
      if (has_q) stage_rows(x_s, sv.qn + rows_off(s, n, nch, 0, K), K, k0, nullptr);
      stage_rows(y_s, sv.w + rows_off(s, n, nch, 0, K), K, k0, nullptr);
      __syncthreads();
#pragma unroll
      for (int i = 0; i < KS / 8; ++i) {
        const int kk = r + 8 * i, k = k0 + kk;
        float x = decay * ds_s[k * (VT + 1) + c];
        if (has_q)
          for (int t = 0; t < R; ++t) x += x_s[t * LDS_ + kk] * o_s[t * (VT + 1) + c];
        for (int t = 0; t < R; ++t) x -= y_s[t * LDS_ + kk] * dd_s[t * (VT + 1) + c];
        if (gr.dstates && vok && k < K) x += gr.dstates[so + (int64_t)v * K + k];
        ds_s[k * (VT + 1) + c] = x;
      }
    }
  }
  __syncthreads();
  if (vok)
    for (int i = 0; i < KM / 8; ++i) {
      const int k = r + 8 * i;
      if (k < K) gr.ds0[(int64_t)s * K * V + (int64_t)k * V + v] = ds_s[k * (VT + 1) + c];
    }
}

// ---------------------------------------------------------------------------
// gdn_chunk_bwd: all per-token gradients of one chunk.
template <typename E, int KM>
__global__ __launch_bounds__(NT) void gdn_chunk_bwd(gpa_gdn_problem p, gpa_gdn_saved sv, gpa_gdn_grads gr,
                                                     int nch) {
  constexpr int NJ = KM / 16;
  extern __shared__ float smem[];
  // Phase A layout: five value-column slices.
  float* pa_do = smem;                      // [R][VT+1]
  float* pa_d = pa_do + R * (VT + 1);       // [R][VT+1]
  float* pa_dd = pa_d + R * (VT + 1);       // [R][VT+1]
  float* pa_h = pa_dd + R * (VT + 1);       // [KM][VT+1]
  float* pa_dh = pa_h + KM * (VT + 1);      // [KM][VT+1]
  // Phase B/C layout (aliases phase A).
  float* pm = smem;                         // [R][LDR]  P then dQK
  float* km = pm + R * LDR;                 // [R][LDR]  A (strictly lower)
  float* tm = km + R * LDR;                 // [R][LDR]  T
  float* dt = tm + R * LDR;                 // [R][LDR]  dT, then dKK sym
  float* xm = dt + R * LDR;                 // [R][LDR]  scratch R x R
  float* a_s = xm + R * LDR;                // [R][LDS_]
  float* b_s = a_s + R * LDS_;              // [R][LDS_]
  constexpr int PHASE_A = 3 * R * (VT + 1) + 2 * KM * (VT + 1);
  constexpr int PHASE_BC = 5 * R * LDR + 2 * R * LDS_;
  constexpr int BASE = PHASE_A > PHASE_BC ? PHASE_A : PHASE_BC;
  float* gam_s = smem + BASE;               // [R]
  float* bet_s = gam_s + R;                 // [R]
  float* dgam_s = bet_s + R;                // [R]
  float* dbet_s = dgam_s + R;               // [R]
  float* red_s = dbet_s + R;                // [4]

  const int n = blockIdx.x, s = blockIdx.y, b = s / p.heads, h = s % p.heads;
  const int K = p.kdim, V = p.vdim, tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
  const bool has_q = p.q.ptr != nullptr && gr.dout.ptr != nullptr;
  const float* kn = sv.kn + rows_off(s, n, nch, 0, K);
  const float* qn = sv.qn + rows_off(s, n, nch, 0, K);
  const float* st = sv.states + state_off(s, n, nch, K, V);
  const float* dh = gr.dhend + state_off(s, n, nch, K, V);
  const float* dl = sv.delta + vc_off(s, n, nch, V);    // value-major [V][R]
  const float* ddl = gr.ddelta + vc_off(s, n, nch, V);
  float* dw = gr.dw + rows_off(s, n, nch, 0, K);

  if (tid < R) {
    gam_s[tid] = sv.gam[rows_off(s, n, nch, 0, 1) + tid];
    bet_s[tid] = sv.beta[rows_off(s, n, nch, 0, 1) + tid];
    dgam_s[tid] = 0.f;
    dbet_s[tid] = 0.f;
  }
  if (tid < 4) red_s[tid] = 0.f;
  __syncthreads();
  const float gc = gam_s[R - 1];

  // ---- Phase A: value-axis contractions against S_n and dS_{n+1}.
  float dq[4][NJ] = {}, dk[4][NJ] = {}, dwr[4][NJ] = {};
  float decay_dot = 0.f;
  for (int v0 = 0; v0 < V; v0 += VT) {
    __syncthreads();
    for (int idx = tid; idx < R * VT; idx += NT) {
      const int r = idx / VT, c = idx % VT, v = v0 + c;
      float o = 0.f;
      if (has_q && v < V) {
        const int t = token_at(p, n, r);
        if (t >= 0) o = op_load<E>(gr.dout, b, h, t, v);
      }
      pa_do[r * (VT + 1) + c] = o;
    }
    for (int idx = tid; idx < R * VT; idx += NT) {
      const int r = idx % R, c = idx / R, v = v0 + c;
      pa_d[r * (VT + 1) + c] = v < V ? dl[(int64_t)v * R + r] : 0.f;
      pa_dd[r * (VT + 1) + c] = v < V ? ddl[(int64_t)v * R + r] : 0.f;
    }
    for (int idx = tid; idx < KM * VT; idx += NT) {
      const int k = idx % KM, c = idx / KM, v = v0 + c;
      const bool ok = k < K && v < V;
      const float hv = ok ? st[(int64_t)v * K + k] : 0.f;
      const float dv = ok ? dh[(int64_t)v * K + k] : 0.f;
      pa_h[k * (VT + 1) + c] = hv;
      pa_dh[k * (VT + 1) + c] = dv;
      decay_dot += hv * dv;
    }
    __syncthreads();
    for (int c = 0; c < VT; ++c) {
      float o[4], d[4], dd[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 4 * ty + i;
        o[i] = pa_do[t * (VT + 1) + c];
        d[i] = pa_d[t * (VT + 1) + c];
        dd[i] = pa_dd[t * (VT + 1) + c];
      }
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int k = tx + 16 * j;
        const float hv = pa_h[k * (VT + 1) + c], dv = pa_dh[k * (VT + 1) + c];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dq[i][j] += o[i] * hv;
          dwr[i][j] -= dd[i] * hv;
          dk[i][j] += d[i] * dv;
        }
      }
    }
  }
  decay_dot = sum64(decay_dot);
  if ((tid & 63) == 0) atomicAdd(&red_s[0], decay_dot);
  // dW to scratch; dQn = e^G dO S^T; dKn = e^{G_C-G} (D dS^T); decay gradients.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 4 * ty + i;
    const float eg = __expf(gam_s[t]), ek = __expf(gc - gam_s[t]);
    float rq = 0.f, rk = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int k = tx + 16 * j;
      if (k < K) dw[(int64_t)t * K + k] = dwr[i][j];
      dq[i][j] *= eg;
      dk[i][j] *= ek;
      if (k < K) {
        if (has_q) rq += dq[i][j] * qn[(int64_t)t * K + k];  // qn is NULL without a query
        rk += dk[i][j] * kn[(int64_t)t * K + k];
      }
    }
    rq = sum16(rq);
    rk = sum16(rk);
    if (tx == 0) {
      atomicAdd(&dgam_s[t], (has_q ? rq : 0.f) - rk);
      atomicAdd(&dgam_s[R - 1], rk);
    }
  }
  if (!has_q) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) dq[i][j] = 0.f;
  }
  __syncthreads();  // phase A LDS free; dW visible below via global (same block)
  if (tid == 0) atomicAdd(&dgam_s[R - 1], __expf(gc) * red_s[0]);

  // ---- Phase B: P path (only when there is a read gradient).
  if (has_q) {
    build_p<KM>(pm, a_s, b_s, qn, kn, gam_s, K);  // pm = P
    // xm = causal dO D^T
    {
      float acc[4][4] = {};
      for (int v0 = 0; v0 < V; v0 += KS) {
        __syncthreads();
        for (int idx = tid; idx < R * KS; idx += NT) {
          const int r = idx / KS, c = idx % KS, v = v0 + c;
          float o = 0.f;
          const int t = token_at(p, n, r);
          if (t >= 0 && v < V) o = op_load<E>(gr.dout, b, h, t, v);
          a_s[r * LDS_ + c] = o;
          b_s[r * LDS_ + c] = v < V ? dl[(int64_t)v * R + r] : 0.f;
        }
        __syncthreads();
        for (int cc = 0; cc < KS; ++cc) {
          float a[4], c2[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) a[i] = a_s[(4 * ty + i) * LDS_ + cc];
#pragma unroll
          for (int j = 0; j < 4; ++j) c2[j] = b_s[(tx + 16 * j) * LDS_ + cc];
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * c2[j];
        }
      }
      // dP -> decay gradients; dQK = dP e^{G_t-G_s} into pm.
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 4 * ty + i;
        float rowsum = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int u = tx + 16 * j;
          const float dp = (u <= t) ? acc[i][j] : 0.f;
          const float pv = pm[t * LDR + u];
          const float g = dp * pv;
          rowsum += g;
          atomicAdd(&dgam_s[u], -g);
          xm[t * LDR + u] = (u <= t) ? dp * __expf(gam_s[t] - gam_s[u]) : 0.f;
        }
        rowsum = sum16(rowsum);
        if (tx == 0) atomicAdd(&dgam_s[t], rowsum);
      }
    }
    __syncthreads();
    // dQn += dQK Kn ; dKn += dQK^T Qn
    for (int k0 = 0; k0 < KM; k0 += KS) {
      __syncthreads();
      stage_rows(a_s, kn, K, k0, nullptr);
      stage_rows(b_s, qn, K, k0, nullptr);
      __syncthreads();
      for (int u = 0; u < R; ++u) {
        float x[4], xt[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[i] = xm[(4 * ty + i) * LDR + u];   // dQK[t][u]
          xt[i] = xm[u * LDR + 4 * ty + i];    // dQK[u][t]
        }
#pragma unroll
        for (int jj = 0; jj < KS / 16; ++jj) {
          const int j = k0 / 16 + jj;
          const float kv = a_s[u * LDS_ + tx + 16 * jj];
          const float qv = b_s[u * LDS_ + tx + 16 * jj];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            dq[i][j] += x[i] * kv;
            dk[i][j] += xt[i] * qv;
          }
        }
      }
    }
  }

  // ---- Phase C: the T = (I+A)^-1 path.
  __syncthreads();
  for (int idx = tid; idx < R * R; idx += NT) tm[(idx / R) * LDR + idx % R] = sv.tri[rows_off(s, n, nch, 0, R) + idx];
  // km = Kn Kn^T;  dt = dD (diag(b) V)^T + dW (diag(b e^G) Kn)^T.
  {
    float kk_acc[4][4] = {}, wk_acc[4][4] = {}, dv_acc[4][4] = {};
    for (int k0 = 0; k0 < KM; k0 += KS) {
      __syncthreads();
      stage_rows(a_s, kn, K, k0, nullptr);
      stage_rows(b_s, dw, K, k0, nullptr);
      __syncthreads();
      for (int kk = 0; kk < KS; ++kk) {
        float a[4], w2[4], c2[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a[i] = a_s[(4 * ty + i) * LDS_ + kk];
          w2[i] = b_s[(4 * ty + i) * LDS_ + kk];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) c2[j] = a_s[(tx + 16 * j) * LDS_ + kk];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            kk_acc[i][j] += a[i] * c2[j];
            wk_acc[i][j] += w2[i] * c2[j];
          }
      }
    }
    for (int v0 = 0; v0 < V; v0 += KS) {
      __syncthreads();
      for (int idx = tid; idx < R * KS; idx += NT) {
        const int r = idx / KS, c = idx % KS, v = v0 + c;
        a_s[r * LDS_ + c] = v < V ? ddl[(int64_t)v * R + r] : 0.f;
        const int t = token_at(p, n, r);
        b_s[r * LDS_ + c] = (t >= 0 && v < V) ? bet_s[r] * op_load<E>(p.v, b, h, t, v) : 0.f;
      }
      __syncthreads();
      for (int cc = 0; cc < KS; ++cc) {
        float a[4], c2[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = a_s[(4 * ty + i) * LDS_ + cc];
#pragma unroll
        for (int j = 0; j < 4; ++j) c2[j] = b_s[(tx + 16 * j) * LDS_ + cc];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) dv_acc[i][j] += a[i] * c2[j];
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 4 * ty + i, u = tx + 16 * j;
        km[t * LDR + u] = kk_acc[i][j];
        dt[t * LDR + u] = dv_acc[i][j] + bet_s[u] * __expf(gam_s[u]) * wk_acc[i][j];
      }
  }
  __syncthreads();
  // xm = dT T^T ; then dA = -(T^T xm), strictly lower, into dt.
  {
    float acc[4][4] = {};
    for (int u = 0; u < R; ++u) {
      float a[4], c2[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = dt[(4 * ty + i) * LDR + u];
#pragma unroll
      for (int j = 0; j < 4; ++j) c2[j] = tm[(tx + 16 * j) * LDR + u];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * c2[j];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) xm[(4 * ty + i) * LDR + tx + 16 * j] = acc[i][j];
  }
  __syncthreads();
  {
    float acc[4][4] = {};
    for (int u = 0; u < R; ++u) {
      float a[4], c2[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = tm[u * LDR + 4 * ty + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) c2[j] = xm[u * LDR + tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * c2[j];
    }
    __syncthreads();  // every row of xm is read above before dKK overwrites it below
    // dA_ts (s<t) = -acc; A_ts = b_t E_ts KK_ts.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 4 * ty + i;
      float rb = 0.f, rg = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int u = tx + 16 * j;
        // Only s < t is live: e^{G_t-G_s} may overflow above the diagonal.
        const bool live = u < t;
        const float da = live ? -acc[i][j] : 0.f;
        const float e = live ? __expf(gam_s[t] - gam_s[u]) : 0.f;
        const float ekk = e * km[t * LDR + u];
        rb += da * ekk;
        const float ga = da * bet_s[t] * ekk;  // dA * A
        rg += ga;
        if (live) atomicAdd(&dgam_s[u], -ga);
        xm[t * LDR + u] = da * bet_s[t] * e;  // dKK (strictly lower)
      }
      rb = sum16(rb);
      rg = sum16(rg);
      if (tx == 0) {
        atomicAdd(&dbet_s[t], rb);
        atomicAdd(&dgam_s[t], rg);
      }
    }
  }
  __syncthreads();
  // dt = dKK + dKK^T (symmetric)
  for (int idx = tid; idx < R * R; idx += NT) {
    const int t = idx / R, u = idx % R;
    dt[t * LDR + u] = xm[t * LDR + u] + xm[u * LDR + t];
  }
  __syncthreads();
  // dKn += dKKsym Kn ;  dKn += diag(b e^G) T^T dW, with beta/decay gradients.
  for (int k0 = 0; k0 < KM; k0 += KS) {
    __syncthreads();
    stage_rows(a_s, kn, K, k0, nullptr);
    stage_rows(b_s, dw, K, k0, nullptr);
    __syncthreads();
    float tdw[4][KS / 16] = {};
    for (int u = 0; u < R; ++u) {
      float x[4], tt[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[i] = dt[(4 * ty + i) * LDR + u];
        tt[i] = tm[u * LDR + 4 * ty + i];  // T[u][s]
      }
#pragma unroll
      for (int jj = 0; jj < KS / 16; ++jj) {
        const float kv = a_s[u * LDS_ + tx + 16 * jj];
        const float wv = b_s[u * LDS_ + tx + 16 * jj];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dk[i][k0 / 16 + jj] += x[i] * kv;
          tdw[i][jj] += tt[i] * wv;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int sr = 4 * ty + i;
      const float eg = __expf(gam_s[sr]);
      float rdot = 0.f;
#pragma unroll
      for (int jj = 0; jj < KS / 16; ++jj) {
        const float kv = a_s[sr * LDS_ + tx + 16 * jj];
        dk[i][k0 / 16 + jj] += bet_s[sr] * eg * tdw[i][jj];
        rdot += kv * tdw[i][jj];
      }
      rdot = sum16(rdot);
      if (tx == 0) {
        atomicAdd(&dbet_s[sr], eg * rdot);
        atomicAdd(&dgam_s[sr], bet_s[sr] * eg * rdot);
      }
    }
  }
  // dV = diag(b) T^T dD ; dbeta += rows of V . (T^T dD)
  for (int v0 = 0; v0 < V; v0 += KS) {
    __syncthreads();
    for (int idx = tid; idx < R * KS; idx += NT) {
      const int r = idx / KS, c = idx % KS, v = v0 + c;
      a_s[r * LDS_ + c] = v < V ? ddl[(int64_t)v * R + r] : 0.f;
      const int t = token_at(p, n, r);
      b_s[r * LDS_ + c] = (t >= 0 && v < V) ? op_load<E>(p.v, b, h, t, v) : 0.f;
    }
    __syncthreads();
    float acc[4][4] = {};
    for (int u = 0; u < R; ++u) {
      float tt[4], c2[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) tt[i] = tm[u * LDR + 4 * ty + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) c2[j] = a_s[u * LDS_ + tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += tt[i] * c2[j];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int sr = 4 * ty + i;
      const int t = token_at(p, n, sr);
      float rdot = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int v = v0 + tx + 16 * j;
        rdot += b_s[sr * LDS_ + tx + 16 * j] * acc[i][j];
        if (t >= 0 && v < V)
          reinterpret_cast<E*>(gr.dv.ptr)[op_base(gr.dv, b, h) + (int64_t)t * gr.dv.st + v] =
              from_f32<E>(bet_s[sr] * acc[i][j]);
      }
      rdot = sum16(rdot);
      if (tx == 0) atomicAdd(&dbet_s[sr], rdot);
    }
  }
  __syncthreads();

  // ---- Phase D: g and beta per token; L2-normalisation backward for q, k.
  if (tid < R) {
    const int t = token_at(p, n, tid);
    if (t >= 0) {
      float acc = 0.f;
      for (int u = tid; u < R; ++u) acc += dgam_s[u];
      float* dg = reinterpret_cast<float*>(gr.dg.ptr);
      float* db = reinterpret_cast<float*>(gr.dbeta.ptr);
      dg[op_base(gr.dg, b, h) + (int64_t)t * gr.dg.st] = acc;
      db[op_base(gr.dbeta, b, h) + (int64_t)t * gr.dbeta.st] = dbet_s[tid];
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * ty + i;
    const int t = token_at(p, n, r);
    for (int which = 0; which < 2; ++which) {
      if (which == 0 && !has_q) {
        if (p.q.ptr && gr.dq.ptr && t >= 0)
          for (int j = 0; j < NJ; ++j) {
            const int k = tx + 16 * j;
            if (k < K) reinterpret_cast<E*>(gr.dq.ptr)[op_base(gr.dq, b, h) + (int64_t)t * gr.dq.st + k] = from_f32<E>(0.f);
          }
        continue;
      }
      const gpa_operand& src = which == 0 ? p.q : p.k;
      const gpa_operand& dst = which == 0 ? gr.dq : gr.dk;
      float ss = 0.f, dot = 0.f, xs[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int k = tx + 16 * j;
        xs[j] = (t >= 0 && k < K) ? op_load<E>(src, b, h, t, k) : 0.f;
        ss += xs[j] * xs[j];
      }
      ss = sum16(ss);
      const float nrm = sqrtf(ss);
      const float den = fmaxf(nrm, 1e-6f);
#pragma unroll
      for (int j = 0; j < NJ; ++j) dot += (xs[j] / den) * (which == 0 ? dq[i][j] : dk[i][j]);
      dot = sum16(dot);
      if (t < 0) continue;
      E* out = reinterpret_cast<E*>(dst.ptr) + op_base(dst, b, h) + (int64_t)t * dst.st;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int k = tx + 16 * j;
        if (k >= K) continue;
        const float g = which == 0 ? dq[i][j] : dk[i][j];
        out[k] = from_f32<E>(nrm > 1e-6f ? (g - (xs[j] / den) * dot) / den : g / 1e-6f);
      }
    }
  }
}

}  // namespace gpa

// ===========================================================================
// Host launchers.
namespace {

using namespace gpa;

int check_problem(const gpa_gdn_problem* p) {
  if (!p) return fail(GPA_HIP_EINVAL, "null problem");
  if (p->batch < 1 || p->heads < 1 || p->tokens < 1)
    return fail(GPA_HIP_EINVAL, "gdn: batch, heads and tokens must be >= 1");
  if (p->chunk < 1 || p->chunk > GPA_CHUNK_ROWS)
    return fail(GPA_HIP_EINVAL, "gdn: chunk must be in [1, 64]");
  if (p->offset < 0 || p->offset >= p->chunk)
    return fail(GPA_HIP_EINVAL, "gdn: offset must be in [0, chunk)");
  if (p->kdim < 1 || p->kdim > GPA_MAX_KDIM) return fail(GPA_HIP_EUNSUPPORTED, "gdn: key width must be in [1, 256]");
  if (p->vdim < 1 || p->vdim > GPA_MAX_VDIM) return fail(GPA_HIP_EUNSUPPORTED, "gdn: value width must be in [1, 1024]");
  if (p->dtype != GPA_DTYPE_F32 && p->dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "gdn: dtype");
  if (!p->k.ptr || !p->v.ptr || !p->g.ptr || !p->beta.ptr) return fail(GPA_HIP_EINVAL, "gdn: null k/v/g/beta");
  if ((int64_t)p->batch * p->heads > 65535) return fail(GPA_HIP_EUNSUPPORTED, "gdn: more than 65535 streams");
  return GPA_HIP_OK;
}

int kmax_for(int k) { return k <= 64 ? 64 : (k <= 128 ? 128 : 256); }

// The bf16 state recurrences run on MFMA when every 16-wide k step is whole.
template <typename E>
bool use_mfma(const gpa_gdn_problem& p) {
  return std::is_same<E, bf16_t>::value && p.kdim % 16 == 0;
}

// Kernels above 64 KiB of dynamic LDS must say so once per instantiation.
template <typename F>
int allow_lds(F kernel, size_t bytes) {
  if (bytes <= 65536) return GPA_HIP_OK;
  const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  return err == hipSuccess ? GPA_HIP_OK : fail(GPA_HIP_EHIP, "hipFuncSetAttribute(max dynamic LDS) failed");
}

// ---- the phases of a forward and a backward (each launches one kernel) ----

template <typename E, int KM>
int fwd_prep(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, int nch, hipStream_t st) {
  return launch_prep_mfma<E, KM>(p, sv, use_mfma<E>(p), nch, st);
}

// A problem whose state recurrence runs on the strip kernels (bf16 MFMA, K <= 128).
template <typename E>
bool strip_path(const gpa_gdn_problem& p) {
  return use_mfma<E>(p) && p.kdim <= 128;
}

// Compute units of the current device (cached per device; 0 if unknown).
int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev] = n;
  }
  return cus[dev];
}

// The strip form of a pack (waves per strip, gdn_strip.h): quarter when its
// workgroups fit on the device's CUs, else split when those fit, else wide;
// each only where every group can take it.
int strip_form(int km, bool fast, bool wide_ok, bool quarter_ok, int quarter_workgroups, int split_workgroups) {
  const int cus = device_cus();
  if (km != 128 || !fast || cus <= 0) return 2;
  if (quarter_ok && quarter_workgroups <= cus) return 4;
  if (wide_ok && split_workgroups > cus) return 1;
  return 2;
}

// The state recurrence of one problem outside a pack.
template <typename E, int KM>
int fwd_state(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, int nch, hipStream_t st) {
  const dim3 block(NT);
  if (strip_path<E>(p)) {
    StripFwdPack pk{};
    pk.n = 1;
    const bool fast = p.kdim == KM && p.vdim % 64 == 0;
    const int nq = strip_form(KM, fast, strip_wide_ok(p), strip_quarter_ok(p), strip_workgroups(p, 4),
                              strip_workgroups(p, 2));
    pk.p[0] = strip_fwd_one(p, sv, nch, 0, nq);
    return launch_state_fwd_strip<KM <= 64 ? 64 : 128>(pk, strip_workgroups(p, nq), fast, nq, st);
  }
  if (use_mfma<E>(p)) return launch_state_fwd_mfma<KM>(p, sv, nch, st);
  const dim3 grid_s((p.vdim + VT - 1) / VT, p.batch * p.heads);
  const size_t lds_state = sizeof(float) * (KM * (VT + 1) + R * LDS_ + R * (VT + 1) + 2 * R);
  if (int rc = allow_lds(gdn_state_fwd<KM>, lds_state)) return rc;
  hipLaunchKernelGGL((gdn_state_fwd<KM>), grid_s, block, lds_state, st, p, sv, nch);
  return GPA_HIP_OK;
}

template <typename E, int KM>
int fwd_out(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, gpa_operand out, int nch, hipStream_t st) {
  if (use_mfma<E>(p) && p.vdim <= GPA_OUT_MFMA_MAX_V) return launch_out_mfma<KM>(p, sv, out, nch, st);
  const dim3 grid_c(nch, p.batch * p.heads), block(NT);
  const size_t lds_out = sizeof(float) * (R * LDR + 2 * R * LDS_ + R);
  hipLaunchKernelGGL((gdn_out_fwd<E, KM>), grid_c, block, lds_out, st, p, sv, out, nch);
  return GPA_HIP_OK;
}

bool has_read(const gpa_gdn_problem& p, const gpa_gdn_grads& gr) { return p.q.ptr && gr.dout.ptr; }

// The grads as the kernels see them: no read gradient, no dd0 / o.
gpa_gdn_grads effective_grads(const gpa_gdn_problem& p, gpa_gdn_grads gr) {
  if (!has_read(p, gr)) {
    gr.dd0 = nullptr;
    gr.o = nullptr;
  }
  return gr;
}

template <typename E, int KM>
int bwd_dd0(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, const gpa_gdn_grads& gr, int nch, hipStream_t st) {
  if (use_mfma<E>(p) && p.vdim <= GPA_OUT_MFMA_MAX_V) return launch_dd0_mfma<KM>(p, sv, gr, nch, st);
  const dim3 grid_c(nch, p.batch * p.heads), block(NT);
  const size_t lds = sizeof(float) * (R * LDR + 2 * R * LDS_ + R);
  hipLaunchKernelGGL((gdn_dd0<E, KM>), grid_c, block, lds, st, p, sv, gr, nch);
  return GPA_HIP_OK;
}

template <typename E, int KM>
int bwd_state(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, const gpa_gdn_grads& gr, int nch, hipStream_t st) {
  const dim3 block(NT);
  if (strip_path<E>(p)) {
    const bool has_q = has_read(p, gr);
    StripBwdPack pk{};
    pk.n = 1;
    const bool fast = p.kdim == KM && p.vdim % 64 == 0, has_inj = gr.dstates != nullptr;
    const int nq = strip_form(KM, fast, strip_wide_ok(p) && !has_inj, strip_quarter_ok(p), strip_workgroups(p, 4),
                              strip_workgroups(p, 2));
    pk.p[0] = strip_bwd_one(p, sv, gr, nch, 0, has_q, nq);
    return launch_state_bwd_strip<KM <= 64 ? 64 : 128>(pk, strip_workgroups(p, nq), fast, has_q, has_inj, nq, st);
  }
  if (use_mfma<E>(p)) return launch_state_bwd_mfma<KM>(p, sv, gr, nch, st);
  const dim3 grid_s((p.vdim + VT - 1) / VT, p.batch * p.heads);
  const size_t lds_state = sizeof(float) * (KM * (VT + 1) + 2 * R * LDS_ + 2 * R * (VT + 1) + 2 * R);
  if (int rc = allow_lds(gdn_state_bwd<E, KM>, lds_state)) return rc;
  hipLaunchKernelGGL((gdn_state_bwd<E, KM>), grid_s, block, lds_state, st, p, sv, gr, nch);
  return GPA_HIP_OK;
}

template <typename E, int KM>
int bwd_chunk(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, const gpa_gdn_grads& gr, int nch, hipStream_t st) {
  // The MFMA chunk kernel keeps 64 x 256 fp32 rows in LDS only for bf16.
  constexpr bool mfma_chunk = !(std::is_same<E, float>::value && KM == 256);
  if (mfma_chunk && p.kdim % 4 == 0) {
    if constexpr (mfma_chunk) return launch_chunk_bwd_mfma<E, KM>(p, sv, gr, nch, st);
  }
  constexpr int PHASE_A = 3 * R * (VT + 1) + 2 * KM * (VT + 1);
  constexpr int PHASE_BC = 5 * R * LDR + 2 * R * LDS_;
  const size_t lds_chunk = sizeof(float) * ((PHASE_A > PHASE_BC ? PHASE_A : PHASE_BC) + 4 * R + 4);
  if (int rc = allow_lds(gdn_chunk_bwd<E, KM>, lds_chunk)) return rc;
  const dim3 grid_c(nch, p.batch * p.heads), block(NT);
  hipLaunchKernelGGL((gdn_chunk_bwd<E, KM>), grid_c, block, lds_chunk, st, p, sv, gr, nch);
  return GPA_HIP_OK;
}

// A phase of problem i, dispatched on its element type and key-width class.
enum class Phase { prep, state, out, dd0, state_bwd, chunk_bwd };

template <typename E, int KM>
int run_phase_km(Phase ph, const gpa_gdn_problem& p, const gpa_gdn_saved& sv, gpa_operand out,
                 const gpa_gdn_grads& gr, int nch, hipStream_t st) {
  switch (ph) {
    case Phase::prep: return fwd_prep<E, KM>(p, sv, nch, st);
    case Phase::state: return fwd_state<E, KM>(p, sv, nch, st);
    case Phase::out: return fwd_out<E, KM>(p, sv, out, nch, st);
    case Phase::dd0: return bwd_dd0<E, KM>(p, sv, gr, nch, st);
    case Phase::state_bwd: return bwd_state<E, KM>(p, sv, gr, nch, st);
    default: return bwd_chunk<E, KM>(p, sv, gr, nch, st);
  }
}

template <typename E>
int run_phase(Phase ph, const gpa_gdn_problem& p, const gpa_gdn_saved& sv, gpa_operand out, const gpa_gdn_grads& gr,
              int nch, hipStream_t st) {
  switch (kmax_for(p.kdim)) {
    case 64: return run_phase_km<E, 64>(ph, p, sv, out, gr, nch, st);
    case 128: return run_phase_km<E, 128>(ph, p, sv, out, gr, nch, st);
    default: return run_phase_km<E, 256>(ph, p, sv, out, gr, nch, st);
  }
}

int phase(Phase ph, const gpa_gdn_problem& p, const gpa_gdn_saved& sv, gpa_operand out, const gpa_gdn_grads& gr,
          hipStream_t st) {
  const int nch = gpa_gdn_nchunks(p.tokens, p.offset, p.chunk);
  return p.dtype == GPA_DTYPE_BF16 ? run_phase<bf16_t>(ph, p, sv, out, gr, nch, st)
                                   : run_phase<float>(ph, p, sv, out, gr, nch, st);
}

bool on_strips(const gpa_gdn_problem& p) { return p.dtype == GPA_DTYPE_BF16 && p.kdim % 16 == 0 && p.kdim <= 128; }
// The 256-key bf16 MFMA state kernels (packed up to GPA_MFMA_MAXP problems).
bool on_mfma256(const gpa_gdn_problem& p) { return p.dtype == GPA_DTYPE_BF16 && p.kdim % 16 == 0 && p.kdim > 128; }

// Forward of n problems: every prep, the state recurrences (the problems on
// the strip kernels of one key-width class in one packed launch, at the
// position of the first of them), every read.
// Part of the groups of a packed call run on a second stream of the device
// (which groups: side_groups).  The state chains leave compute units idle
// (one strip workgroup per CU; 32-96 workgroups of the 256-key kernel), so
// the other stream's kernels fill them.  Each group's phases (prep or dd0,
// state, out or chunk backward) run in order on its stream, between a fork
// event at the start of the call and a join at its end.  The side stream and
// its events are created on first use per device and kept for the process
// (default priority).  The enqueue sequence fork -> launches -> join runs
// under one mutex, so concurrent calls never interleave their event records.
// Timed calls and calls under graph capture stay on one stream.
struct SideStream {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
constexpr int kSideDevices = 64;
std::mutex g_side_mutex;
SideStream g_side[kSideDevices];

bool capturing(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone;
}

// Locks g_side_mutex into `lock`, creates the side stream of st's device if
// needed, and makes it wait for everything st has enqueued so far.
int side_fork(hipStream_t st, SideStream*& out, std::unique_lock<std::mutex>& lock) {
  hipDevice_t dev = 0;
  if (hipStreamGetDevice(st, &dev) != hipSuccess) return fail(GPA_HIP_EHIP, "gdn: hipStreamGetDevice failed");
  if (dev < 0 || dev >= kSideDevices) return fail(GPA_HIP_EUNSUPPORTED, "gdn: device index above 63");
  lock = std::unique_lock<std::mutex>(g_side_mutex);
  SideStream& sd = g_side[dev];
  if (!sd.s) {
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) return fail(GPA_HIP_EHIP, "gdn: hipGetDevice failed");
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return fail(GPA_HIP_EHIP, "gdn: hipSetDevice failed");
    SideStream made;
    hipError_t e = hipStreamCreateWithFlags(&made.s, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&made.fork, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&made.join, hipEventDisableTiming);
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess) return fail(GPA_HIP_EHIP, "gdn: creating the side stream failed");
    sd = made;
  }
  if (hipEventRecord(sd.fork, st) != hipSuccess || hipStreamWaitEvent(sd.s, sd.fork, 0) != hipSuccess)
    return fail(GPA_HIP_EHIP, "gdn: side stream fork failed");
  out = &sd;
  return GPA_HIP_OK;
}

int side_join(hipStream_t st, const SideStream& sd) {
  if (hipEventRecord(sd.join, sd.s) != hipSuccess || hipStreamWaitEvent(st, sd.join, 0) != hipSuccess)
    return fail(GPA_HIP_EHIP, "gdn: side stream join failed");
  return GPA_HIP_OK;
}

// Holds the side stream of one call from its fork to its join.  The join
// (the caller's stream waits for everything enqueued on the side stream) is
// recorded on every return path once a fork has happened, so that a call that
// fails part-way still leaves the side work ordered before later work on the
// caller's stream; the mutex is released after the join.
struct SideScope {
  hipStream_t st;
  SideStream* sd = nullptr;
  std::unique_lock<std::mutex> lock;
  explicit SideScope(hipStream_t s) : st(s) {}
  SideScope(const SideScope&) = delete;
  SideScope& operator=(const SideScope&) = delete;
  ~SideScope() {
    if (sd) (void)side_join(st, *sd);
  }
  int join() {
    SideStream* s = sd;
    sd = nullptr;
    return s ? side_join(st, *s) : GPA_HIP_OK;
  }
};

// Which groups of the call run on the side stream: the 256-key groups when
// the call also has others; else, for a call of strip groups only (a level's
// A/B pair), the second half of the groups, each half in its own strip pack,
// so that one half's prep or out phase overlaps the other half's state chain
// (only while all their strip workgroups fit on the device's CUs at once;
// beyond that the groups stay in one pack, which takes the wide form).
// Returns whether any group goes there (never for timed or captured calls).
bool side_groups(const gpa_gdn_problem* ps, int n, const gpa_timing* tm, hipStream_t st, bool (&side)[GPA_GDN_MAX_PACK]) {
  bool mf = false, other = false, strips = true;
  for (int i = 0; i < n; ++i) {
    (on_mfma256(ps[i]) ? mf : other) = true;
    strips = strips && on_strips(ps[i]);
    side[i] = false;
  }
  if (tm || capturing(st)) return false;
  if (mf && other) {
    for (int i = 0; i < n; ++i) side[i] = on_mfma256(ps[i]);
    return true;
  }
  if (strips && n >= 2) {
    int wg = 0;
    for (int i = 0; i < n; ++i) wg += strip_workgroups(ps[i], 2);
    const int cus = device_cus();
    if (cus <= 0 || wg > cus) return false;
    for (int i = n / 2; i < n; ++i) side[i] = true;
    return true;
  }
  return false;
}

int launch_forward_many(const gpa_gdn_problem* ps, const gpa_gdn_saved* svs, const gpa_operand* outs, int n,
                        gpa_timing* tm, hipStream_t st) {
  const gpa_gdn_grads none{};
  SideScope side(st);
  bool on_side[GPA_GDN_MAX_PACK];
  if (side_groups(ps, n, tm, st, on_side))
    if (int rc = side_fork(st, side.sd, side.lock)) return rc;
  auto stream_of = [&](int i) { return side.sd && on_side[i] ? side.sd->s : st; };
  for (int i = 0; i < n; ++i) {
    mark(tm, st);
    if (int rc = phase(Phase::prep, ps[i], svs[i], outs[i], none, stream_of(i))) return rc;
  }
  bool done[GPA_GDN_MAX_PACK] = {};
  for (int i = 0; i < n; ++i) {
    if (done[i]) continue;
    mark(tm, st);
    if (on_mfma256(ps[i])) {
      MfmaPack pk{};
      int total = 0;
      bool fast = true;
      for (int j = i; j < n && pk.n < GPA_MFMA_MAXP; ++j) {
        if (done[j] || !on_mfma256(ps[j]) || on_side[j] != on_side[i]) continue;
        pk.p[pk.n] = ps[j];
        pk.sv[pk.n] = svs[j];
        pk.nch[pk.n] = gpa_gdn_nchunks(ps[j].tokens, ps[j].offset, ps[j].chunk);
        pk.nvb[pk.n] = (ps[j].vdim + 63) / 64;
        pk.wg0[pk.n++] = total;
        total += mfma_state_workgroups(ps[j]);
        fast = fast && ps[j].kdim == 256 && ps[j].vdim % 64 == 0;
        done[j] = true;
      }
      if (int rc = launch_state_fwd_mfma_pack<256>(pk, total, fast, stream_of(i))) return rc;
      continue;
    }
    if (!on_strips(ps[i])) {
      if (int rc = phase(Phase::state, ps[i], svs[i], outs[i], none, stream_of(i))) return rc;
      continue;
    }
    const int km = kmax_for(ps[i].kdim);
    int members[GPA_GDN_MAX_PACK], nm = 0, split = 0, quarter = 0;
    bool fast = true, wide_ok = true, quarter_ok = true;
    for (int j = i; j < n; ++j) {
      if (done[j] || !on_strips(ps[j]) || kmax_for(ps[j].kdim) != km || on_side[j] != on_side[i]) continue;
      members[nm++] = j;
      split += strip_workgroups(ps[j], 2);
      quarter += strip_workgroups(ps[j], 4);
      fast = fast && ps[j].kdim == km && ps[j].vdim % 64 == 0;
      wide_ok = wide_ok && strip_wide_ok(ps[j]);
      quarter_ok = quarter_ok && strip_quarter_ok(ps[j]);
      done[j] = true;
    }
    const int nq = strip_form(km, fast, wide_ok, quarter_ok, quarter, split);
    StripFwdPack pk{};
    int total = 0;
    for (int m = 0; m < nm; ++m) {
      const int j = members[m];
      const int nch = gpa_gdn_nchunks(ps[j].tokens, ps[j].offset, ps[j].chunk);
      pk.p[pk.n++] = strip_fwd_one(ps[j], svs[j], nch, total, nq);
      total += strip_workgroups(ps[j], nq);
    }
    const int rc = km <= 64 ? launch_state_fwd_strip<64>(pk, total, fast, nq, stream_of(i))
                            : launch_state_fwd_strip<128>(pk, total, fast, nq, stream_of(i));
    if (rc) return rc;
  }
  // the out phase of each group follows its state pack on the same stream
  for (int i = 0; i < n; ++i) {
    if (!ps[i].q.ptr || !outs[i].ptr) continue;
    mark(tm, st);
    if (int rc = phase(Phase::out, ps[i], svs[i], outs[i], none, stream_of(i))) return rc;
  }
  if (int rc = side.join()) return rc;
  mark(tm, st);
  return check_launch("gdn_forward");
}

// Backward of n problems: every dd0, the state recurrences (packed per
// key-width class, read gradient and state injection), every chunk kernel.
int launch_backward_many(const gpa_gdn_problem* ps, const gpa_gdn_saved* svs, const gpa_gdn_grads* grs, int n,
                         gpa_timing* tm, hipStream_t st) {
  const gpa_operand none{};
  gpa_gdn_grads gr[GPA_GDN_MAX_PACK];
  for (int i = 0; i < n; ++i) gr[i] = effective_grads(ps[i], grs[i]);
  SideScope side(st);
  bool on_side[GPA_GDN_MAX_PACK];
  if (side_groups(ps, n, tm, st, on_side))
    if (int rc = side_fork(st, side.sd, side.lock)) return rc;
  auto stream_of = [&](int i) { return side.sd && on_side[i] ? side.sd->s : st; };
  for (int i = 0; i < n; ++i) {
    if (!has_read(ps[i], gr[i])) continue;
    mark(tm, st);
    if (int rc = phase(Phase::dd0, ps[i], svs[i], none, gr[i], stream_of(i))) return rc;
  }
  bool done[GPA_GDN_MAX_PACK] = {};
  for (int i = 0; i < n; ++i) {
    if (done[i]) continue;
    mark(tm, st);
    const bool hq = has_read(ps[i], gr[i]), hi = gr[i].dstates != nullptr;
    if (on_mfma256(ps[i])) {
      MfmaPack pk{};
      int total = 0;
      bool fast = true;
      for (int j = i; j < n && pk.n < GPA_MFMA_MAXP; ++j) {
        if (done[j] || !on_mfma256(ps[j]) || has_read(ps[j], gr[j]) != hq || (gr[j].dstates != nullptr) != hi ||
            on_side[j] != on_side[i])
          continue;
        pk.p[pk.n] = ps[j];
        pk.sv[pk.n] = svs[j];
        pk.gr[pk.n] = gr[j];
        pk.nch[pk.n] = gpa_gdn_nchunks(ps[j].tokens, ps[j].offset, ps[j].chunk);
        pk.nvb[pk.n] = (ps[j].vdim + 63) / 64;
        pk.wg0[pk.n++] = total;
        total += mfma_state_workgroups(ps[j]);
        fast = fast && ps[j].kdim == 256 && ps[j].vdim % 64 == 0;
        done[j] = true;
      }
      if (int rc = launch_state_bwd_mfma_pack<256>(pk, total, fast, hq, hi, stream_of(i))) return rc;
      continue;
    }
    if (!on_strips(ps[i])) {
      if (int rc = phase(Phase::state_bwd, ps[i], svs[i], none, gr[i], stream_of(i))) return rc;
      continue;
    }
    const int km = kmax_for(ps[i].kdim);
    int members[GPA_GDN_MAX_PACK], nm = 0, split = 0, quarter = 0;
    bool fast = true, wide_ok = !hi, quarter_ok = true;
    for (int j = i; j < n; ++j) {
      if (done[j] || !on_strips(ps[j]) || kmax_for(ps[j].kdim) != km || has_read(ps[j], gr[j]) != hq ||
          (gr[j].dstates != nullptr) != hi || on_side[j] != on_side[i])
        continue;
      members[nm++] = j;
      split += strip_workgroups(ps[j], 2);
      quarter += strip_workgroups(ps[j], 4);
      fast = fast && ps[j].kdim == km && ps[j].vdim % 64 == 0;
      wide_ok = wide_ok && strip_wide_ok(ps[j]);
      quarter_ok = quarter_ok && strip_quarter_ok(ps[j]);
      done[j] = true;
    }
    const int nq = strip_form(km, fast, wide_ok, quarter_ok, quarter, split);
    StripBwdPack pk{};
    int total = 0;
    for (int m = 0; m < nm; ++m) {
      const int j = members[m];
      const int nch = gpa_gdn_nchunks(ps[j].tokens, ps[j].offset, ps[j].chunk);
      pk.p[pk.n++] = strip_bwd_one(ps[j], svs[j], gr[j], nch, total, hq, nq);
      total += strip_workgroups(ps[j], nq);
    }
    const int rc = km <= 64 ? launch_state_bwd_strip<64>(pk, total, fast, hq, hi, nq, stream_of(i))
                            : launch_state_bwd_strip<128>(pk, total, fast, hq, hi, nq, stream_of(i));
    if (rc) return rc;
  }
  // the chunk phase of each group follows its state pack on the same stream
  for (int i = 0; i < n; ++i) {
    mark(tm, st);
    if (int rc = phase(Phase::chunk_bwd, ps[i], svs[i], none, gr[i], stream_of(i))) return rc;
  }
  if (int rc = side.join()) return rc;
  mark(tm, st);
  return check_launch("gdn_backward");
}

}  // namespace

static int path_of(const gpa_gdn_problem* p) { return p->dtype == GPA_DTYPE_BF16 && p->kdim % 16 == 0 ? 1 : 0; }

static int check_saved(const gpa_gdn_problem* p, const gpa_gdn_saved* sv) {
  if (!sv || !sv->kn || !sv->u || !sv->delta || !sv->tri || !sv->gam || !sv->beta || !sv->states || !sv->final)
    return fail(GPA_HIP_EINVAL, "gdn: a saved buffer is null");
  if (p->q.ptr && !sv->qn) return fail(GPA_HIP_EINVAL, "gdn: q given without qn");
  if (path_of(p)) {
    if (!sv->wrow || !sv->wcol || !sv->krow || !sv->kcol || (p->q.ptr && !sv->qcol))
      return fail(GPA_HIP_EINVAL, "gdn: the MFMA path needs the fragment buffers");
  } else if (!sv->w) {
    return fail(GPA_HIP_EINVAL, "gdn: the FMA path needs w");
  }
  return GPA_HIP_OK;
}

extern "C" int32_t gpa_gdn_path(const gpa_gdn_problem* problem) { return problem ? path_of(problem) : 0; }

extern "C" int32_t gpa_gdn_nchunks(int32_t tokens, int32_t offset, int32_t chunk) {
  if (tokens < 1 || chunk < 1 || chunk > GPA_CHUNK_ROWS || offset < 0 || offset >= chunk) return 0;
  return (offset + tokens + chunk - 1) / chunk;
}

extern "C" int gpa_gdn_forward(const gpa_gdn_problem* problem, const gpa_gdn_saved* saved, gpa_operand out,
                               gpa_timing* timing, hipStream_t stream) {
  int rc = check_problem(problem);
  if (rc) return rc;
  if (int rc2 = check_saved(problem, saved)) return rc2;
  if (problem->q.ptr && !out.ptr) return fail(GPA_HIP_EINVAL, "gdn_forward: q given without out");
  if (timing) timing->launched = 0;
  return launch_forward_many(problem, saved, &out, 1, timing, stream);
}

extern "C" int gpa_gdn_forward_many(const gpa_gdn_problem* problems, const gpa_gdn_saved* saved,
                                    const gpa_operand* outs, int32_t n, gpa_timing* timing, hipStream_t stream) {
  if (!problems || !saved || !outs || n < 1 || n > GPA_GDN_MAX_PACK)
    return fail(GPA_HIP_EINVAL, "gdn_forward_many: 1 to GPA_GDN_MAX_PACK problems with saved buffers and outs");
  for (int i = 0; i < n; ++i) {
    if (int rc = check_problem(&problems[i])) return rc;
    if (int rc = check_saved(&problems[i], &saved[i])) return rc;
    if (problems[i].q.ptr && !outs[i].ptr) return fail(GPA_HIP_EINVAL, "gdn_forward_many: q given without out");
  }
  if (timing) timing->launched = 0;
  return launch_forward_many(problems, saved, outs, n, timing, stream);
}

extern "C" int gpa_gdn_backward(const gpa_gdn_problem* problem, const gpa_gdn_saved* saved,
                                const gpa_gdn_grads* grads, gpa_timing* timing, hipStream_t stream) {
  int rc = check_problem(problem);
  if (rc) return rc;
  if (!grads) return fail(GPA_HIP_EINVAL, "gdn_backward: null grads");
  if (int rc2 = check_saved(problem, saved)) return rc2;
  if (!grads->ddelta || !grads->dhend || !grads->dw || !grads->dk.ptr || !grads->dv.ptr || !grads->dg.ptr ||
      !grads->dbeta.ptr || !grads->ds0)
    return fail(GPA_HIP_EINVAL, "gdn_backward: a gradient buffer is null");
  if (problem->q.ptr && grads->dout.ptr && (!grads->dd0 || !grads->o || !grads->dq.ptr))
    return fail(GPA_HIP_EINVAL, "gdn_backward: read gradient needs dd0, o and dq");
  if (timing) timing->launched = 0;
  return launch_backward_many(problem, saved, grads, 1, timing, stream);
}

extern "C" int gpa_gdn_backward_many(const gpa_gdn_problem* problems, const gpa_gdn_saved* saved,
                                     const gpa_gdn_grads* grads, int32_t n, gpa_timing* timing, hipStream_t stream) {
  if (!problems || !saved || !grads || n < 1 || n > GPA_GDN_MAX_PACK)
    return fail(GPA_HIP_EINVAL, "gdn_backward_many: 1 to GPA_GDN_MAX_PACK problems with saved buffers and grads");
  for (int i = 0; i < n; ++i) {
    const gpa_gdn_problem* problem = &problems[i];
    const gpa_gdn_grads* g = &grads[i];
    if (int rc = check_problem(problem)) return rc;
    if (int rc = check_saved(problem, &saved[i])) return rc;
    if (!g->ddelta || !g->dhend || !g->dw || !g->dk.ptr || !g->dv.ptr || !g->dg.ptr || !g->dbeta.ptr || !g->ds0)
      return fail(GPA_HIP_EINVAL, "gdn_backward_many: a gradient buffer is null");
    if (problem->q.ptr && g->dout.ptr && (!g->dd0 || !g->o || !g->dq.ptr))
      return fail(GPA_HIP_EINVAL, "gdn_backward_many: read gradient needs dd0, o and dq");
  }
  if (timing) timing->launched = 0;
  return launch_backward_many(problems, saved, grads, n, timing, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free forward (gpa_gdn_scan_noalloc).  The intermediates that
// gpa_gdn_forward takes from its caller live in `scratch`, a static device
// array of GPA_NOALLOC_SCRATCH_BYTES that every device the library runs on
// holds until the process ends.  Host code never passes `scratch` itself to a
// kernel (in host code the name is only a stand-in for the symbol): the
// device address comes from hipGetSymbolAddress, taken once per device, with
// that device current, on the first call there.  The forward kernels write
// every element of the intermediates they later read, so nothing needs
// clearing between calls.  All calls on one device share its array: calls
// that overlap in time on one device (two streams, two threads) race.
namespace {

static __device__ __align__(256) unsigned char scratch[GPA_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];  // per device, set once under the mutex

int scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(GPA_HIP_EHIP, "gdn_scan_noalloc: hipGetDevice failed");
  if (dev < 0 || dev >= kMaxDevices) return fail(GPA_HIP_EUNSUPPORTED, "gdn_scan_noalloc: device index above 63");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr) {
      char buf[160];
      snprintf(buf, sizeof buf, "gdn_scan_noalloc: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(err));
      return fail(GPA_HIP_EHIP, buf);
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return GPA_HIP_OK;
}

// Carve the forward's intermediates (the sizes gpa_gdn_saved documents in
// include/gpa_hip.h) from `base` in 256-byte aligned pieces; returns the bytes
// used.  With base == 0 it only measures.
uint64_t carve_saved(const gpa_gdn_problem& p, uintptr_t base, gpa_gdn_saved* sv) {
  const uint64_t nch = gpa_gdn_nchunks(p.tokens, p.offset, p.chunk);
  const uint64_t chunks = (uint64_t)p.batch * p.heads * nch, rows = chunks * R;
  const uint64_t K = p.kdim, V = p.vdim, k16 = K / 16, rb = (K + 31) / 32;
  const bool mfma = path_of(&p) == 1, has_q = p.q.ptr != nullptr;
  uint64_t at = 0;
  auto take = [&](uint64_t bytes) -> void* {
    if (!bytes) return nullptr;
    void* ptr = reinterpret_cast<void*>(base + at);
    at += (bytes + 255) / 256 * 256;
    return ptr;
  };
  const uint64_t f = sizeof(float), h = 2;  // float32, bf16 element sizes
  sv->kn = static_cast<float*>(take(rows * K * f));
  sv->qn = static_cast<float*>(take(has_q ? rows * K * f : 0));
  sv->w = static_cast<float*>(take(mfma ? 0 : rows * K * f));
  sv->u = static_cast<float*>(take(rows * (mfma ? (uint64_t)ufrag_v(p.vdim) : V) * f));
  sv->delta = static_cast<float*>(take(rows * V * f));
  sv->tri = static_cast<float*>(take(rows * R * f));
  sv->gam = static_cast<float*>(take(rows * f));
  sv->beta = static_cast<float*>(take(rows * f));
  sv->states = static_cast<float*>(take(chunks * V * K * f));
  sv->final = nullptr;  // the caller's output
  sv->wrow = take(mfma ? chunks * 2 * k16 * 64 * 16 * h : 0);
  sv->wcol = take(mfma ? chunks * rb * 4 * 64 * 16 * h : 0);
  sv->krow = take(mfma ? chunks * 2 * k16 * 64 * 8 * h : 0);
  sv->kcol = take(mfma ? chunks * rb * 4 * 64 * 8 * h : 0);
  sv->qcol = take(mfma && has_q ? chunks * rb * 4 * 64 * 8 * h : 0);
  return at;
}

}  // namespace

extern "C" int gpa_gdn_scan_noalloc(const gpa_gdn_problem* problem, gpa_operand out, float* final_state,
                                    hipStream_t stream) {
  int rc = check_problem(problem);
  if (rc) return rc;
  if (!final_state) return fail(GPA_HIP_EINVAL, "gdn_scan_noalloc: final_state is null");
  if (problem->q.ptr && !out.ptr) return fail(GPA_HIP_EINVAL, "gdn_scan_noalloc: q given without out");
  gpa_gdn_saved sv{};
  const uint64_t need = carve_saved(*problem, 0, &sv);
  if (need > (uint64_t)GPA_NOALLOC_SCRATCH_BYTES) {
    char buf[200];
    snprintf(buf, sizeof buf,
             "gdn_scan_noalloc: the problem needs %llu bytes of scratch, above the %llu-byte maximum "
             "(fewer streams or tokens per call)",
             (unsigned long long)need, (unsigned long long)GPA_NOALLOC_SCRATCH_BYTES);
    return fail(GPA_HIP_EINVAL, buf);
  }
  void* base = nullptr;
  if ((rc = scratch_address(&base))) return rc;
  carve_saved(*problem, reinterpret_cast<uintptr_t>(base), &sv);
  sv.final = final_state;
  return launch_forward_many(problem, &sv, &out, 1, nullptr, stream);
}
