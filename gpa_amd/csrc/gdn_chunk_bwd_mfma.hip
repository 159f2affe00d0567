// Chunk-parallel GDN backward on fp32 MFMA (v_mfma_f32_32x32x2f32 and
// v_mfma_f32_16x16x4f32), one block per (chunk, stream), 4 waves.
//
// Within a chunk (rows t, u < 64, keys k, values v) the forward solved
//   D = T Rhs,   Rhs = diag(b) V - diag(b e^G) Kn S_n,   T = (I + A)^-1,
// so with dD the full gradient of D and dS the gradient of the chunk-end
// state (both from the reverse recurrence):
//   Y   = T^T dD                       gradient of Rhs;  dV = diag(b) Y
//   X   = dD D^T,  dA = -(T^T X)       strictly lower (dT = dD Rhs^T, dA = -T^T dT T^T)
//   dP  = dO D^T                       causal, P = e^{G_t-G_u} Qn Kn^T
//   dQn = e^G dO S_n^T + dQK Kn
//   dKn = e^{G_C-G} D dS^T - diag(b e^G) Y S_n^T + dQK^T Qn + (dKK + dKK^T) Kn
// plus the gate gradients of every e^G factor and b, then the L2
// normalisation backward of q and k.  The contraction over the value axis is
// streamed through LDS in 16-value slices; each wave owns fixed 32x32 output
// tiles and keeps them in accumulators for the whole kernel.
//
// Operand feeding.  A 32x32x2 MFMA step takes one A and one B value per lane:
// A(row l%32, c), B(c, col l%32) with c = 2 s + l/32.  This file instead
// feeds, over four steps s = 0..3, contraction index c0 + s with
// c0 = 8 g + 4 (l/32): the same 8 indices of group g, permuted.  A lane then
// needs four consecutive contraction values of one row or column, which is
// one 16-byte LDS read when the contraction axis is contiguous (ld_c) and
// four conflict-free scalar reads when the row axis is (ld_x).  The
// accumulator of a 32x32 tile holds, in lane l register r, row
// 8 (r/4) + 4 (l/32) + r%4 and column l%32.
#include <hip/hip_runtime.h>

#include "gdn_common.h"

namespace gpa {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace {

__device__ __forceinline__ void mma8(f32x16& c, f32x4 a, f32x4 b) {
  c = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b.x, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b.y, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b.z, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b.w, c, 0, 0, 0);
}

// 16x16x4 with the same permutation: lane quarter q = l/16 feeds c0 + s, c0 = 16 g + 4 q.
__device__ __forceinline__ void mma16(f32x4& c, f32x4 a, f32x4 b) {
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, c, 0, 0, 0);
}

// Element (x, c0 + s), s = 0..3, of a matrix stored with c contiguous ...
__device__ __forceinline__ f32x4 ld_c(const float* m, int ld, int x, int c0) {
  return *reinterpret_cast<const f32x4*>(m + x * ld + c0);
}
// ... or with x contiguous.
__device__ __forceinline__ f32x4 ld_x(const float* m, int ld, int x, int c0) {
  return f32x4{m[c0 * ld + x], m[(c0 + 1) * ld + x], m[(c0 + 2) * ld + x], m[(c0 + 3) * ld + x]};
}

// A copy of a uniform value the compiler cannot see through: values derived
// from it inside a loop are not hoisted out of the loop (where they would
// occupy registers for its whole length).
template <typename T>
__device__ __forceinline__ T opaque(T x) {
  asm volatile("" : "+s"(x));
  return x;
}

__device__ __forceinline__ int acc_row(int r, int half) { return 8 * (r >> 2) + 4 * half + (r & 3); }

// Sums of each of a lane's 16 accumulator-row values over the 32 lanes of its
// half-wave, by recursive halving (16 exchanges instead of 16 x 5).  Every
// lane returns the sum for register index sum_index(lane).
__device__ __forceinline__ float tile_row_sum(float (&v)[16], int lane) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const bool up = lane & 16;
    const float send = up ? v[j] : v[j + 8], keep = up ? v[j + 8] : v[j];
    v[j] = keep + __shfl_xor(send, 16);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool up = lane & 8;
    const float send = up ? v[j] : v[j + 4], keep = up ? v[j + 4] : v[j];
    v[j] = keep + __shfl_xor(send, 8);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const bool up = lane & 4;
    const float send = up ? v[j] : v[j + 2], keep = up ? v[j + 2] : v[j];
    v[j] = keep + __shfl_xor(send, 4);
  }
  {
    const bool up = lane & 2;
    const float send = up ? v[0] : v[1], keep = up ? v[1] : v[0];
    v[0] = keep + __shfl_xor(send, 2);
  }
  return v[0] + __shfl_xor(v[0], 1);
}
__device__ __forceinline__ int sum_index(int lane) {
  return 8 * ((lane >> 4) & 1) + 4 * ((lane >> 3) & 1) + 2 * ((lane >> 2) & 1) + ((lane >> 1) & 1);
}

}  // namespace

// LDS plan (floats).  One key panel (KM <= 128): the R x R matrices reuse the
// staging area once the value loop is done; two panels keep dQK and dKK apart.
template <int KM>
struct ChunkBwdLayout {
  static constexpr int KP = KM < 128 ? KM : 128;  // key panel
  static constexpr int NP = KM / KP;
  static constexpr int VS = 16;                   // value slice
  static constexpr int LDO = VS + 4, LT = R + 4, LS = KP + 4, KSL = 32, LKN = KSL + 4;
  // value-loop staging
  static constexpr int DO = 0, VV = DO + R * LDO, D = VV + R * LDO, DD = D + VS * LT, Y = DD + VS * LT,
                       S = Y + VS * LT, DS = S + VS * LS, V_END = DS + VS * LS;
  // key-loop staging (P, KK)
  static constexpr int QK = 0, KK = QK + R * LKN, K_END = KK + R * LKN;
  static constexpr int RR1 = 2 * R * LT;  // xm + dQK inside the staging area (one panel)
  static constexpr int STAGE = V_END > RR1 ? (V_END > K_END ? V_END : K_END) : (RR1 > K_END ? RR1 : K_END);
  static constexpr int T_OFF = 0;
  static constexpr int OWN = NP == 1 ? 0 : 2 * R * LT;  // separate dQK, dKK
  static constexpr int STAGE_OFF = R * LT + OWN;
  static constexpr int XM_OFF = STAGE_OFF;
  static constexpr int DQK_OFF = NP == 1 ? STAGE_OFF + R * LT : R * LT;
  static constexpr int DKK_OFF = NP == 1 ? STAGE_OFF : 2 * R * LT;
  static constexpr int SC_OFF = STAGE_OFF + STAGE;
  static constexpr int TOTAL = SC_OFF + 9 * R + 4;
};

template <typename E, int KM>
__global__ __launch_bounds__(NT, 1) void gdn_chunk_bwd_mfma(gpa_gdn_problem p, gpa_gdn_saved sv,
                                                                          gpa_gdn_grads gr, int nch) {
  using L = ChunkBwdLayout<KM>;
  constexpr int KP = L::KP, NP = L::NP, VS = L::VS, LDO = L::LDO, LT = L::LT, LS = L::LS, KSL = L::KSL,
                LKN = L::LKN;
  constexpr int NTW = KP / 64;        // R x KP output tiles per wave
  constexpr int SQ = VS * KP / 4 / NT;  // float4 of S per thread per slice
  static_assert(SQ >= 1 && VS * R / 4 == NT && R * VS == 4 * NT, "staging shape");
  extern __shared__ __align__(16) float smem[];
  float* tm = smem + L::T_OFF;
  float* stage = smem + L::STAGE_OFF;
  float* do_s = stage + L::DO;
  float* vv_s = stage + L::VV;
  float* d_s = stage + L::D;
  float* dd_s = stage + L::DD;
  float* y_s = stage + L::Y;
  float* s_s = stage + L::S;
  float* ds_s = stage + L::DS;
  float* qk_s = stage + L::QK;
  float* kk_s = stage + L::KK;
  float* xm = smem + L::XM_OFF;
  float* dqk = smem + L::DQK_OFF;
  float* dkk = smem + L::DKK_OFF;
  float* gam_s = smem + L::SC_OFF;
  float* bet_s = gam_s + R;
  float* dgam_s = bet_s + R;
  float* dbet_s = dgam_s + R;
  float* qss_s = dbet_s + R;
  float* qxg_s = qss_s + R;
  float* kss_s = qxg_s + R;
  float* kxg_s = kss_s + R;
  int* tok_s = reinterpret_cast<int*>(kxg_s + R);  // token of each row (-1: void)
  float* red_s = kxg_s + 2 * R;

  const int n = blockIdx.x, s = blockIdx.y, b = s / p.heads, h = s % p.heads;
  const int K = p.kdim, V = p.vdim, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, hh = lane >> 5;
  const bool has_q = p.q.ptr != nullptr && gr.dout.ptr != nullptr;
  const float* kn0 = sv.kn + rows_off(s, n, nch, 0, K);
  const float* qn0 = has_q ? sv.qn + rows_off(s, n, nch, 0, K) : nullptr;
  const float* st = sv.states + state_off(s, n, nch, K, V);
  const float* dh = gr.dhend + state_off(s, n, nch, K, V);
  const float* dl = sv.delta + vc_off(s, n, nch, V);
  const float* ddl = gr.ddelta + vc_off(s, n, nch, V);
  const float* tri = sv.tri + rows_off(s, n, nch, 0, R);

  if (tid < R) {
    gam_s[tid] = sv.gam[rows_off(s, n, nch, 0, 1) + tid];
    bet_s[tid] = sv.beta[rows_off(s, n, nch, 0, 1) + tid];
    dgam_s[tid] = dbet_s[tid] = 0.f;
    qss_s[tid] = qxg_s[tid] = kss_s[tid] = kxg_s[tid] = 0.f;
    tok_s[tid] = token_at(p, n, tid);
  }
  if (tid < 4) red_s[tid] = 0.f;
  for (int i = tid; i < R * R / 4; i += NT) {
    const int t = i / (R / 4), c = 4 * (i % (R / 4));
    *reinterpret_cast<f32x4*>(tm + t * LT + c) = *reinterpret_cast<const f32x4*>(tri + t * R + c);
  }
  __syncthreads();
  const float gc = gam_s[R - 1];

  // Output tiles: R x KP tiles m < NTW at rows 32 rt(m), panel columns 32 kt;
  // the R x R tile at (32 rr, 32 ru).
  const int kt = NTW == 2 ? wave : (wave & 1);
  const int rr = wave >> 1, ru = wave & 1;
  auto tile_rt = [&](int m) { return NTW == 2 ? m : (wave >> 1); };

  f32x16 dp = {}, xt = {};
  // dQn, dKn of the current panel (the last one after the loop); earlier
  // panels are parked unnormalised in dq/dk and re-read by the same lanes.
  f32x16 dq[NTW], dka[NTW], dkw[NTW];
  float ddot = 0.f;                 // this thread's share of <S_n, dS>
  const int nsl = (V + VS - 1) / VS;

#pragma unroll 1
  for (int panel = 0; panel < NP; ++panel) {
    const int kb = panel * KP;
    const int K = opaque(p.kdim);
    const float* kn = opaque(kn0);
    const float* qn = opaque(qn0);
#pragma unroll
    for (int m = 0; m < NTW; ++m) dq[m] = dka[m] = dkw[m] = f32x16{};

    // ---- value loop: register prefetch of slice sl+1 while slice sl is in LDS.
    f32x4 rs[SQ], rds[SQ], rd, rdd;
    float rdo[4], rv[4];
    auto fetch = [&](int v0) {
#pragma unroll
      for (int i = 0; i < SQ; ++i) {
        const int idx = tid + NT * i, vr = idx / (KP / 4), c = 4 * (idx % (KP / 4));
        const int v = v0 + vr, k = kb + c;
        const bool ok = v < V && k < K;
        rs[i] = ok ? *reinterpret_cast<const f32x4*>(st + (int64_t)v * K + k) : f32x4{};
        rds[i] = ok ? *reinterpret_cast<const f32x4*>(dh + (int64_t)v * K + k) : f32x4{};
      }
      {
        const int vr = tid / (R / 4), c = 4 * (tid % (R / 4)), v = v0 + vr;
        rd = v < V ? *reinterpret_cast<const f32x4*>(dl + (int64_t)v * R + c) : f32x4{};
        rdd = v < V ? *reinterpret_cast<const f32x4*>(ddl + (int64_t)v * R + c) : f32x4{};
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int idx = tid + NT * i, t = idx / VS, v = v0 + idx % VS;
        const int tok = token_at(p, n, t);
        const bool ok = tok >= 0 && v < V;
        rdo[i] = (has_q && ok) ? op_load<E>(gr.dout, b, h, tok, v) : 0.f;
        rv[i] = (panel == 0 && ok) ? op_load<E>(p.v, b, h, tok, v) : 0.f;
      }
    };
    auto stash = [&]() {
#pragma unroll
      for (int i = 0; i < SQ; ++i) {
        const int idx = tid + NT * i, vr = idx / (KP / 4), c = 4 * (idx % (KP / 4));
        *reinterpret_cast<f32x4*>(s_s + vr * LS + c) = rs[i];
        *reinterpret_cast<f32x4*>(ds_s + vr * LS + c) = rds[i];
        ddot += rs[i].x * rds[i].x + rs[i].y * rds[i].y + rs[i].z * rds[i].z + rs[i].w * rds[i].w;
      }
      {
        const int vr = tid / (R / 4), c = 4 * (tid % (R / 4));
        *reinterpret_cast<f32x4*>(d_s + vr * LT + c) = rd;
        *reinterpret_cast<f32x4*>(dd_s + vr * LT + c) = rdd;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int idx = tid + NT * i, t = idx / VS, c = idx % VS;
        do_s[t * LDO + c] = rdo[i];
        vv_s[t * LDO + c] = rv[i];
      }
    };

    fetch(0);
    stash();
    __syncthreads();
    for (int sl = 0; sl < nsl; ++sl) {
      const int v0 = sl * VS;
      if (sl + 1 < nsl) fetch(v0 + VS);
      // Y slice: rows 16 wave .. +15, the 16 values of the slice (16x16x4).
      {
        const int tq = lane & 15, q = lane >> 4;
        f32x4 y = {};
#pragma unroll
        for (int g = 0; g < R / 16; ++g) {
          const int c0 = 16 * g + 4 * q;
          mma16(y, ld_x(tm, LT, 16 * wave + tq, c0), ld_c(dd_s, LT, tq, c0));
        }
        *reinterpret_cast<f32x4*>(y_s + tq * LT + 16 * wave + 4 * q) = y;
        if (panel == 0) {
          float part[4];
          const int v = v0 + tq;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = 16 * wave + 4 * q + r;
            const int tok = token_at(p, n, t);
            if (tok >= 0 && v < V)
              reinterpret_cast<float*>(gr.dv.ptr)[op_base(gr.dv, b, h) + (int64_t)tok * gr.dv.st + v] = bet_s[t] * y[r];
            part[r] = vv_s[t * LDO + tq] * y[r];
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float x = part[r];
            x += __shfl_xor(x, 8);
            x += __shfl_xor(x, 4);
            x += __shfl_xor(x, 2);
            x += __shfl_xor(x, 1);
            if (tq == 0) atomicAdd(&dbet_s[16 * wave + 4 * q + r], x);
          }
        }
      }
      __syncthreads();
#pragma unroll
      for (int g = 0; g < VS / 8; ++g) {
        const int c0 = 8 * g + 4 * hh;
        const f32x4 bs = ld_x(s_s, LS, 32 * kt + li, c0);
        const f32x4 bds = ld_x(ds_s, LS, 32 * kt + li, c0);
#pragma unroll
        for (int m = 0; m < NTW; ++m) {
          const int row = 32 * tile_rt(m) + li;
          if (has_q) mma8(dq[m], ld_c(do_s, LDO, row, c0), bs);
          mma8(dka[m], ld_x(d_s, LT, row, c0), bds);
          mma8(dkw[m], ld_x(y_s, LT, row, c0), bs);
        }
        if (panel == 0) {
          const f32x4 bu = ld_x(d_s, LT, 32 * ru + li, c0);
          if (has_q) mma8(dp, ld_c(do_s, LDO, 32 * rr + li, c0), bu);
          mma8(xt, ld_x(dd_s, LT, 32 * rr + li, c0), bu);
        }
      }
      __syncthreads();
      if (sl + 1 < nsl) {
        stash();
        __syncthreads();
      }
    }

    // ---- value-axis terms: scale rows, gate gradients, merge the Y term into dKn.
    {
      const int k = kb + 32 * kt + li;
      const bool kin = k < K;
      float rk_total = 0.f;
#pragma unroll
      for (int m = 0; m < NTW; ++m) {
        const int rt = tile_rt(m);
        float pq[16], pk[16], pw[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = 32 * rt + acc_row(r, hh);
          const float eg = __expf(gam_s[t]), ek = __expf(gc - gam_s[t]);
          const float kv = kin ? kn[(int64_t)t * K + k] : 0.f;
          if (has_q) {
            dq[m][r] *= eg;
            pq[r] = (kin ? qn[(int64_t)t * K + k] : 0.f) * dq[m][r];
          } else {
            pq[r] = 0.f;
          }
          dka[m][r] *= ek;
          pk[r] = kv * dka[m][r];
          const float w = -dkw[m][r];
          pw[r] = kv * w;
          dka[m][r] += bet_s[t] * eg * w;
        }
        const float sq = tile_row_sum(pq, lane), sk = tile_row_sum(pk, lane), sw = tile_row_sum(pw, lane);
        if ((lane & 1) == 0) {
          const int t = 32 * rt + acc_row(sum_index(lane), hh);
          const float eg = __expf(gam_s[t]);
          atomicAdd(&dgam_s[t], sq - sk + bet_s[t] * eg * sw);
          atomicAdd(&dbet_s[t], eg * sw);
          rk_total += sk;
        }
      }
      rk_total = sum64(rk_total);
      if (lane == 0) atomicAdd(&dgam_s[R - 1], rk_total);
    }

    if (panel == 0) {
      // ---- P and KK on this wave's R x R tile: contraction over all keys.
      f32x16 pt = {}, kkt = {};
      for (int k0 = 0; k0 < KM; k0 += KSL) {
        __syncthreads();
        for (int i = tid; i < R * KSL; i += NT) {
          const int r = i / KSL, c = i % KSL, k = k0 + c;
          qk_s[r * LKN + c] = (has_q && k < K) ? qn[(int64_t)r * K + k] : 0.f;
          kk_s[r * LKN + c] = k < K ? kn[(int64_t)r * K + k] : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < KSL / 8; ++g) {
          const int c0 = 8 * g + 4 * hh;
          const f32x4 bk = ld_c(kk_s, LKN, 32 * ru + li, c0);
          if (has_q) mma8(pt, ld_c(qk_s, LKN, 32 * rr + li, c0), bk);
          mma8(kkt, ld_c(kk_s, LKN, 32 * rr + li, c0), bk);
        }
      }
      __syncthreads();
      // ---- dP: gate gradients and dQK; X to LDS.
      {
        const int u = 32 * ru + li;
        float prow[16], pcol = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = 32 * rr + acc_row(r, hh);
          const bool live = u <= t;
          const float e = live ? __expf(gam_s[t] - gam_s[u]) : 0.f;
          const float dpv = (has_q && live) ? dp[r] : 0.f;
          const float g = dpv * e * pt[r];
          prow[r] = g;
          pcol += g;
          dqk[t * LT + u] = dpv * e;
          xm[t * LT + u] = xt[r];
        }
        const float srow = tile_row_sum(prow, lane);
        if ((lane & 1) == 0) atomicAdd(&dgam_s[32 * rr + acc_row(sum_index(lane), hh)], srow);
        pcol += __shfl_xor(pcol, 32);
        if (hh == 0) atomicAdd(&dgam_s[u], -pcol);
      }
      __syncthreads();
      // ---- dA = -(T^T X), strictly lower: b, gate and dKK.
      {
        f32x16 da = {};
#pragma unroll
        for (int g = 0; g < R / 8; ++g) {
          const int c0 = 8 * g + 4 * hh;
          mma8(da, ld_x(tm, LT, 32 * rr + li, c0), ld_x(xm, LT, 32 * ru + li, c0));
        }
        __syncthreads();  // xm is read by every wave before dKK overwrites it
        const int u = 32 * ru + li;
        float rb[16], rg[16], gcol = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = 32 * rr + acc_row(r, hh);
          const bool live = u < t;  // e^{G_t-G_u} may overflow above the diagonal
          const float dav = live ? -da[r] : 0.f;
          const float e = live ? __expf(gam_s[t] - gam_s[u]) : 0.f;
          const float ekk = e * kkt[r];
          rb[r] = dav * ekk;
          const float ga = dav * bet_s[t] * ekk;
          rg[r] = ga;
          gcol += ga;
          dkk[t * LT + u] = dav * bet_s[t] * e;
        }
        const float sb = tile_row_sum(rb, lane), sg = tile_row_sum(rg, lane);
        if ((lane & 1) == 0) {
          const int t = 32 * rr + acc_row(sum_index(lane), hh);
          atomicAdd(&dbet_s[t], sb);
          atomicAdd(&dgam_s[t], sg);
        }
        gcol += __shfl_xor(gcol, 32);
        if (hh == 0) atomicAdd(&dgam_s[u], -gcol);
      }
      __syncthreads();
    }

    // ---- position-axis terms: dQn += dQK Kn; dKn += dQK^T Qn + (dKK + dKK^T) Kn.
    {
      const int k = kb + 32 * kt + li;
      const bool kin = k < K;
      f32x4 bk[R / 8], bq[R / 8];
#pragma unroll
      for (int g = 0; g < R / 8; ++g) {
        const int c0 = 8 * g + 4 * hh;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          bk[g][e] = kin ? kn[(int64_t)(c0 + e) * K + k] : 0.f;
          bq[g][e] = (has_q && kin) ? qn[(int64_t)(c0 + e) * K + k] : 0.f;
        }
      }
#pragma unroll
      for (int m = 0; m < NTW; ++m) {
        const int row = 32 * tile_rt(m) + li;
#pragma unroll
        for (int g = 0; g < R / 8; ++g) {
          const int c0 = 8 * g + 4 * hh;
          if (has_q) {
            mma8(dq[m], ld_c(dqk, LT, row, c0), bk[g]);
            mma8(dka[m], ld_x(dqk, LT, row, c0), bq[g]);
          }
          mma8(dka[m], ld_c(dkk, LT, row, c0) + ld_x(dkk, LT, row, c0), bk[g]);
        }
      }
    }

    // ---- normalisation backward, part 1: row sums of x^2 and x . g.
    {
      const int k = kb + 32 * kt + li;
      const bool kin = k < K;
#pragma unroll
      for (int m = 0; m < NTW; ++m) {
        const int rt = tile_rt(m);
        float a[16], c[16], aq[16], cq[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = 32 * rt + acc_row(r, hh);
          const int tok = tok_s[t];  // read from LDS inside the panel loop: keeps row offsets out of registers
          const bool ok = tok >= 0 && kin;
          const float xk = ok ? op_load<E>(p.k, b, h, tok, k) : 0.f;
          a[r] = xk * xk;
          c[r] = xk * dka[m][r];
          const float xq = (ok && has_q) ? op_load<E>(p.q, b, h, tok, k) : 0.f;
          aq[r] = xq * xq;
          cq[r] = xq * dq[m][r];
        }
        const float sa = tile_row_sum(a, lane), sc = tile_row_sum(c, lane);
        float saq = 0.f, scq = 0.f;
        if (has_q) {
          saq = tile_row_sum(aq, lane);
          scq = tile_row_sum(cq, lane);
        }
        if ((lane & 1) == 0) {
          const int t = 32 * rt + acc_row(sum_index(lane), hh);
          atomicAdd(&kss_s[t], sa);
          atomicAdd(&kxg_s[t], sc);
          if (has_q) {
            atomicAdd(&qss_s[t], saq);
            atomicAdd(&qxg_s[t], scq);
          }
        }
        if (panel + 1 < NP) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int tok = tok_s[32 * rt + acc_row(r, hh)];
            if (tok < 0 || !kin) continue;
            if (has_q && gr.dq.ptr)
              reinterpret_cast<float*>(gr.dq.ptr)[op_base(gr.dq, b, h) + (int64_t)tok * gr.dq.st + k] = dq[m][r];
            reinterpret_cast<float*>(gr.dk.ptr)[op_base(gr.dk, b, h) + (int64_t)tok * gr.dk.st + k] = dka[m][r];
          }
        }
      }
    }
  }

  ddot = sum64(ddot);
  if (lane == 0) atomicAdd(&red_s[0], ddot);
  __syncthreads();
  if (tid == 0) dgam_s[R - 1] += __expf(gc) * red_s[0];

  // ---- normalisation backward, part 2: write dq, dk (every panel).
#pragma unroll 1
  for (int panel = 0; panel < NP; ++panel) {
    const int k = panel * KP + 32 * kt + li;
    if (k >= K) continue;
#pragma unroll
    for (int m = 0; m < NTW; ++m) {
      const int rt = tile_rt(m);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = 32 * rt + acc_row(r, hh);
        const int tok = token_at(p, n, t);
        if (tok < 0) continue;
        for (int which = 0; which < 2; ++which) {
          const gpa_operand& src = which == 0 ? p.q : p.k;
          const gpa_operand& dst = which == 0 ? gr.dq : gr.dk;
          if (!src.ptr || !dst.ptr) continue;
          float* out = reinterpret_cast<float*>(dst.ptr) + op_base(dst, b, h) + (int64_t)tok * dst.st;
          if (which == 0 && !has_q) {
            out[k] = 0.f;
            continue;
          }
          const float g = panel + 1 < NP ? out[k] : (which == 0 ? dq[m][r] : dka[m][r]);
          const float ss = which == 0 ? qss_s[t] : kss_s[t], xg = which == 0 ? qxg_s[t] : kxg_s[t];
          const float nrm = sqrtf(ss), den = fmaxf(nrm, 1e-6f);
          const float xh = op_load<E>(src, b, h, tok, k) / den;
          out[k] = nrm > 1e-6f ? (g - xh * (xg / den)) / den : g / 1e-6f;
        }
      }
    }
  }
  __syncthreads();
  if (tid < R) {
    const int tok = token_at(p, n, tid);
    if (tok >= 0) {
      float acc = 0.f;
      for (int u = tid; u < R; ++u) acc += dgam_s[u];
      reinterpret_cast<float*>(gr.dg.ptr)[op_base(gr.dg, b, h) + (int64_t)tok * gr.dg.st] = acc;
      reinterpret_cast<float*>(gr.dbeta.ptr)[op_base(gr.dbeta, b, h) + (int64_t)tok * gr.dbeta.st] = dbet_s[tid];
    }
  }
}

template <typename E, int KM>
int launch_chunk_bwd_mfma(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, const gpa_gdn_grads& gr, int nch,
                          hipStream_t st) {
  const size_t lds = sizeof(float) * ChunkBwdLayout<KM>::TOTAL;
  if (lds > 65536) {
    const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(gdn_chunk_bwd_mfma<E, KM>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (err != hipSuccess) return fail(GPA_HIP_EHIP, "hipFuncSetAttribute(max dynamic LDS) failed");
  }
  hipLaunchKernelGGL((gdn_chunk_bwd_mfma<E, KM>), dim3(nch, p.batch * p.heads), dim3(NT), lds, st, p, sv, gr, nch);
  return GPA_HIP_OK;
}

template int launch_chunk_bwd_mfma<float, 64>(const gpa_gdn_problem&, const gpa_gdn_saved&, const gpa_gdn_grads&,
                                              int, hipStream_t);
template int launch_chunk_bwd_mfma<float, 128>(const gpa_gdn_problem&, const gpa_gdn_saved&, const gpa_gdn_grads&,
                                               int, hipStream_t);
template int launch_chunk_bwd_mfma<float, 256>(const gpa_gdn_problem&, const gpa_gdn_saved&, const gpa_gdn_grads&,
                                               int, hipStream_t);
template int launch_chunk_bwd_mfma<bf16_t, 64>(const gpa_gdn_problem&, const gpa_gdn_saved&, const gpa_gdn_grads&,
                                               int, hipStream_t);
template int launch_chunk_bwd_mfma<bf16_t, 128>(const gpa_gdn_problem&, const gpa_gdn_saved&, const gpa_gdn_grads&,
                                                int, hipStream_t);
template int launch_chunk_bwd_mfma<bf16_t, 256>(const gpa_gdn_problem&, const gpa_gdn_saved&, const gpa_gdn_grads&,
                                                int, hipStream_t);

}  // namespace gpa
