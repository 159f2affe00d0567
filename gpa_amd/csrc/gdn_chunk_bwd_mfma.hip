// Chunk-parallel GDN backward on fp32 MFMA (v_mfma_f32_32x32x2f32 and
// v_mfma_f32_16x16x4f32), one block per (chunk, stream), 8 waves.
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
// tiles and keeps them in accumulators for the whole kernel.  The block
// recomputes the row norms of its raw keys and queries (the same sums as the
// forward's normalisation) and keeps x/|x| in LDS: its rounding is the matrix
// operand Kn/Qn, the unrounded value the input of the normalisation backward.
//
// Operand feeding and accumulator layouts: mfma_tiles.h.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "mfma_tiles.h"

namespace gpa {

// LDS plan (floats).  The R x R matrices reuse the staging area once the value
// loop is done.  Up to 128 keys, x/|x| is kept unrounded (fp32); with 256 keys
// (bf16 only) it is kept rounded, as bf16, and the normalisation backward
// re-reads the raw rows.
template <typename E, int KM>
struct ChunkBwdLayout {
  static constexpr bool XR = KM > 128;
  // Value slice: 32 values for bf16 activations up to 128 keys (half the
  // dependent load rounds of the value loop, twice the bytes in flight per
  // round; the LDS still fits), else 16.
  static constexpr int VS = std::is_same<E, bf16_t>::value && KM <= 128 ? 32 : 16;
  // bf16 activations: each 16 values of a slice run as one 32x32x16 step
  // (BFV), with dO rows read as 8-byte pairs (LDO a multiple of 4)
  static constexpr bool BFV = std::is_same<E, bf16_t>::value;
  static constexpr int LDO = VS + 4, LT = R + 4, LS = KM + 4;
  static constexpr int LX = XR ? KM + 8 : KM + 4;  // row stride of x/|x| (bf16 elements when XR)
  static constexpr int XF = XR ? R * LX / 2 : R * LX;
  static constexpr int EQ = R * LDO * (int)sizeof(E) / 4;  // floats of one [R][LDO] activation tile
  // value-loop staging
  static constexpr int DO = 0, VV = DO + EQ, D = VV + EQ, DD = D + VS * LT, Y = DD + VS * LT, S = Y + VS * LT,
                       DS = S + VS * LS, V_END = DS + VS * LS;
  static constexpr int RR1 = 2 * R * LT;  // xm (dKK) + dQK
  static constexpr int STAGE = RR1 > V_END ? RR1 : V_END;
  static constexpr int T_OFF = 0, XK_OFF = R * LT, XQ_OFF = XK_OFF + XF, STAGE_OFF = XQ_OFF + XF;
  static constexpr int XM_OFF = STAGE_OFF, DQK_OFF = STAGE_OFF + R * LT, DKK_OFF = STAGE_OFF;
  static constexpr int SC_OFF = STAGE_OFF + STAGE;
  static constexpr int TOTAL = SC_OFF + 13 * R + 4;
  static constexpr size_t BYTES = sizeof(float) * TOTAL;
};

constexpr int CB_WAVES = 8, CB_NT = 64 * CB_WAVES;  // threads of a chunk-backward block

template <typename E, int KM>
__global__ __launch_bounds__(CB_NT, 1) void gdn_chunk_bwd_mfma(gpa_gdn_problem p, gpa_gdn_saved sv,
                                                              gpa_gdn_grads gr, int nch) {
  using L = ChunkBwdLayout<E, KM>;
  constexpr bool XR = L::XR;
  static_assert(!XR || std::is_same<E, bf16_t>::value, "rounded x/|x| needs bf16 activations");
  constexpr int VS = L::VS, LDO = L::LDO, LT = L::LT, LS = L::LS, LX = L::LX;
  constexpr bool BFV = L::BFV;
  constexpr int NW = CB_WAVES, NTH = CB_NT, KT = KM / 32;
  constexpr int NTW = KT >= 4 ? KT / 4 : 1;  // R x K output tiles per owning wave
  // Per-slice staging counts (float4 of S/dS, of D/dD; elements of dO/V) and
  // their per-thread shares; entries past a count are loaded from index 0
  // (always valid) and not stored.
  constexpr int SC = VS * KM / 4, DC = VS * R / 4, OC = R * VS;
  constexpr int SQ = (SC + NTH - 1) / NTH, DQ = (DC + NTH - 1) / NTH, OQ = (OC + NTH - 1) / NTH;
  static_assert(VS % 16 == 0, "value slice");
  extern __shared__ __align__(16) float smem[];
  float* tm = smem + L::T_OFF;
  float* xk_s = smem + L::XK_OFF;  // x/|x| (fp32), or its bf16 rounding when XR
  float* xq_s = smem + L::XQ_OFF;
  bf16_t* xkb = reinterpret_cast<bf16_t*>(xk_s);
  bf16_t* xqb = reinterpret_cast<bf16_t*>(xq_s);
  float* stage = smem + L::STAGE_OFF;
  E* do_s = reinterpret_cast<E*>(stage + L::DO);
  E* vv_s = reinterpret_cast<E*>(stage + L::VV);
  float* d_s = stage + L::D;
  float* dd_s = stage + L::DD;
  float* y_s = stage + L::Y;
  float* s_s = stage + L::S;
  float* ds_s = stage + L::DS;
  float* xm = smem + L::XM_OFF;
  float* dqk = smem + L::DQK_OFF;
  float* dkk = smem + L::DKK_OFF;
  float* gam_s = smem + L::SC_OFF;
  float* bet_s = gam_s + R;
  float* dgam_s = bet_s + R;
  float* dbet_s = dgam_s + R;
  float* qnrm_s = dbet_s + R;  // |q_t|, |k_t| of the raw rows
  float* knrm_s = qnrm_s + R;
  float* qdot_s = knrm_s + R;  // sum_k x/|x| . dX of the rows
  float* kdot_s = qdot_s + R;
  float* eg_s = kdot_s + R;   // e^{G_t}
  float* ek_s = eg_s + R;     // e^{G_C - G_t}
  float* qrd_s = ek_s + R;    // 1 / max(|q_t|, 1e-6), 1 / max(|k_t|, 1e-6)
  float* krd_s = qrd_s + R;
  int* tok_s = reinterpret_cast<int*>(krd_s + R);  // token of each row (-1: void)
  float* red_s = krd_s + 2 * R;

  const int n = blockIdx.x, s = blockIdx.y, b = s / p.heads, h = s % p.heads;
  const int K = p.kdim, V = p.vdim, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, hh = lane >> 5;
  const bool has_q = p.q.ptr != nullptr && gr.dout.ptr != nullptr;
  const float* st = sv.states + state_off(s, n, nch, K, V);
  const float* dh = gr.dhend + state_off(s, n, nch, K, V);
  const float* dl = sv.delta + vc_off(s, n, nch, V);
  const float* ddl = gr.ddelta + vc_off(s, n, nch, V);
  const float* tri = sv.tri + rows_off(s, n, nch, 0, R);
  // x/|x| rounded to the activation type (the matrix operand Kn, Qn) ...
  auto kr = [&](int t, int k) { return XR ? to_f32(xkb[t * LX + k]) : round_as<E>(xk_s[t * LX + k]); };
  auto qr = [&](int t, int k) { return XR ? to_f32(xqb[t * LX + k]) : round_as<E>(xq_s[t * LX + k]); };

  if (tid < R) {
    gam_s[tid] = sv.gam[rows_off(s, n, nch, 0, 1) + tid];
    bet_s[tid] = sv.beta[rows_off(s, n, nch, 0, 1) + tid];
    dgam_s[tid] = dbet_s[tid] = 0.f;
    qdot_s[tid] = kdot_s[tid] = 0.f;
    tok_s[tid] = token_at(p, n, tid);
  }
  if (tid < 4) red_s[tid] = 0.f;
  {
    // the triangular inverse: every load issued before the first store
    constexpr int TQ = (R * R / 4 + NTH - 1) / NTH;
    f32x4 tv[TQ];
#pragma unroll
    for (int j = 0; j < TQ; ++j) {
      const int i = tid + NTH * j, ic = i < R * R / 4 ? i : 0;
      tv[j] = *reinterpret_cast<const f32x4*>(tri + 4 * ic);
    }
#pragma unroll
    for (int j = 0; j < TQ; ++j) {
      const int i = tid + NTH * j;
      if ((R * R / 4) % NTH != 0 && i >= R * R / 4) continue;
      *reinterpret_cast<f32x4*>(tm + (i / (R / 4)) * LT + 4 * (i % (R / 4))) = tv[j];
    }
  }
  // Row norms of the raw keys and queries, summed in the forward's order, and
  // x/|x| for every key column.  Every load of the wave is issued (at a clamped
  // address, from a stand-in operand when there is no query) before the first
  // use.
  const gpa_operand& qsrc = has_q ? p.q : p.k;
  {
    constexpr int NI = KM / 64, NR = R / NW;
    float xk[NR][NI], xq[NR][NI];
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      const int tok = token_at(p, n, wave + NW * j), tt = tok >= 0 ? tok : 0;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int d = lane + 64 * i, dd = d < K ? d : 0;
        xk[j][i] = op_load<E>(p.k, b, h, tt, dd);
        xq[j][i] = op_load<E>(qsrc, b, h, tt, dd);
      }
    }
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      const int r = wave + NW * j, tok = token_at(p, n, r);
      float sk = 0.f, sq = 0.f;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const bool ok = tok >= 0 && lane + 64 * i < K;
        xk[j][i] = ok ? xk[j][i] : 0.f;
        xq[j][i] = (ok && has_q) ? xq[j][i] : 0.f;
        sk += xk[j][i] * xk[j][i];
        sq += xq[j][i] * xq[j][i];
      }
      const float nk = sqrtf(sum64(sk)), nq = sqrtf(sum64(sq));
      if (lane == 0) {
        knrm_s[r] = nk;
        qnrm_s[r] = nq;
        krd_s[r] = 1.f / fmaxf(nk, 1e-6f);
        qrd_s[r] = 1.f / fmaxf(nq, 1e-6f);
      }
      const float dk = fmaxf(nk, 1e-6f), dq = fmaxf(nq, 1e-6f);
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int c = r * LX + lane + 64 * i;
        if (XR) {
          xkb[c] = from_f32<bf16_t>(xk[j][i] / dk);
          xqb[c] = from_f32<bf16_t>(xq[j][i] / dq);
        } else {
          xk_s[c] = xk[j][i] / dk;
          xq_s[c] = xq[j][i] / dq;
        }
      }
    }
  }
  __syncthreads();
  const float gc = gam_s[R - 1];
  if (tid < R) {
    eg_s[tid] = __expf(gam_s[tid]);
    ek_s[tid] = __expf(gc - gam_s[tid]);
  }

  // Tiles.  Waves below 2 KT own NTW R x K output tiles of dQn, dKn and the
  // Y S^T term, tile m at rows 32 rt(m), columns 32 kt; the R x R tile
  // (32 rr, 32 ru) is shared by wave w (dP, P: waves 0-3) and wave w + 4
  // (X, KK, dA: waves 4-7).
  const bool own = wave < 2 * KT;
  const int kt = own ? (NTW == 2 ? wave : wave % KT) : 0;
  auto tile_rt = [&](int m) { return NTW == 2 ? m : (own ? wave / KT : 0); };
  const int rr = (wave & 3) >> 1, ru = wave & 1;
  const bool grp_p = wave < 4;

  f32x16 dp = {};  // dP on waves 0-3, X on waves 4-7
  f32x16 dq[NTW], dka[NTW], dkw[NTW];
#pragma unroll
  for (int m = 0; m < NTW; ++m) dq[m] = dka[m] = dkw[m] = f32x16{};
  float ddot = 0.f;  // this thread's share of <S_n, dS>
  const int nsl = (V + VS - 1) / VS;

  // ---- value loop: register prefetch of slice sl+1 while slice sl is in LDS.
  // fetch() only issues loads (at a clamped, always valid address); the masks
  // of void or out-of-range entries are applied in stash(), after the MFMA
  // work of the current slice, so the loads stay in flight meanwhile.  With
  // 256 keys the prefetch registers would spill (their reloads cost more than
  // the overlap gains): each slice is loaded just before its use.
  constexpr bool PREFETCH = !XR;
  {
    const gpa_operand& dosrc = has_q ? gr.dout : p.v;  // stand-in of the same shape when there is no read
    f32x4 rs[SQ], rds[SQ], rd[DQ], rdd[DQ];
    E rdo[OQ], rv[OQ];
    int vnext = 0;
    auto fetch = [&](int v0) {
      vnext = v0;
#pragma unroll
      for (int i = 0; i < SQ; ++i) {
        const int idx0 = tid + NTH * i, idx = idx0 < SC ? idx0 : 0;
        const int vr = idx / (KM / 4), c = 4 * (idx % (KM / 4));
        const int v = v0 + vr;
        const int64_t o = (v < V && c < K) ? (int64_t)v * K + c : 0;
        rs[i] = *reinterpret_cast<const f32x4*>(st + o);
        rds[i] = *reinterpret_cast<const f32x4*>(dh + o);
      }
#pragma unroll
      for (int i = 0; i < DQ; ++i) {
        const int idx0 = tid + NTH * i, idx = idx0 < DC ? idx0 : 0;
        const int vr = idx / (R / 4), c = 4 * (idx % (R / 4)), v = v0 + vr;
        const int64_t o = v < V ? (int64_t)v * R + c : 0;
        rd[i] = *reinterpret_cast<const f32x4*>(dl + o);
        rdd[i] = *reinterpret_cast<const f32x4*>(ddl + o);
      }
#pragma unroll
      for (int i = 0; i < OQ; ++i) {
        const int idx0 = tid + NTH * i, idx = idx0 < OC ? idx0 : 0;
        const int t = idx / VS, v = v0 + idx % VS;
        const int tok = tok_s[t];
        const bool ok = tok >= 0 && v < V;
        const int tt = ok ? tok : 0, vv = ok ? v : 0;
        rdo[i] = op_raw<E>(dosrc, b, h, tt, vv);
        rv[i] = op_raw<E>(p.v, b, h, tt, vv);
      }
    };
    auto stash = [&]() {
      const int v0 = vnext;
#pragma unroll
      for (int i = 0; i < SQ; ++i) {
        const int idx = tid + NTH * i;
        if (SC % NTH != 0 && idx >= SC) continue;
        const int vr = idx / (KM / 4), c = 4 * (idx % (KM / 4));
        const bool ok = v0 + vr < V && c < K;
        const f32x4 a = ok ? rs[i] : f32x4{}, d = ok ? rds[i] : f32x4{};
        *reinterpret_cast<f32x4*>(s_s + vr * LS + c) = a;
        *reinterpret_cast<f32x4*>(ds_s + vr * LS + c) = d;
        ddot += a.x * d.x + a.y * d.y + a.z * d.z + a.w * d.w;
      }
#pragma unroll
      for (int i = 0; i < DQ; ++i) {
        const int idx = tid + NTH * i;
        if (DC % NTH != 0 && idx >= DC) continue;
        const int vr = idx / (R / 4), c = 4 * (idx % (R / 4));
        const bool ok = v0 + vr < V;
        *reinterpret_cast<f32x4*>(d_s + vr * LT + c) = ok ? rd[i] : f32x4{};
        *reinterpret_cast<f32x4*>(dd_s + vr * LT + c) = ok ? rdd[i] : f32x4{};
      }
#pragma unroll
      for (int i = 0; i < OQ; ++i) {
        const int idx = tid + NTH * i;
        if (OC % NTH != 0 && idx >= OC) continue;
        const int t = idx / VS, c = idx % VS;
        const bool ok = tok_s[t] >= 0 && v0 + c < V;
        do_s[t * LDO + c] = (ok && has_q) ? rdo[i] : from_f32<E>(0.f);
        vv_s[t * LDO + c] = ok ? rv[i] : from_f32<E>(0.f);
      }
    };

    if (PREFETCH) {
      fetch(0);
      stash();
      __syncthreads();
    }
    for (int sl = 0; sl < nsl; ++sl) {
      const int v0 = sl * VS;
      if (!PREFETCH) {
        fetch(v0);
        stash();
        __syncthreads();
      } else if (sl + 1 < nsl) {
        fetch(v0 + VS);
      }
      // Y tile (16x16x4): rows 16 (w % 4) .. +15, slice values 16 (w / 4) .. +15.
      if (wave < 4 * (VS / 16)) {
        const int tq = lane & 15, q = lane >> 4, t0 = 16 * (wave & 3), j = wave >> 2;
        f32x4 y = {};
#pragma unroll
        for (int g = 0; g < R / 16; ++g) {
          const int c0 = 16 * g + 4 * q;
          mma16(y, ld_x(tm, LT, t0 + tq, c0), ld_c(dd_s, LT, 16 * j + tq, c0));
        }
        *reinterpret_cast<f32x4*>(y_s + (16 * j + tq) * LT + t0 + 4 * q) = y;
        float part[4];
        const int v = v0 + 16 * j + tq;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = t0 + 4 * q + r;
          const int tok = tok_s[t];
          if (tok >= 0 && v < V)
            reinterpret_cast<E*>(gr.dv.ptr)[op_base(gr.dv, b, h) + (int64_t)tok * gr.dv.st + v] = from_f32<E>(bet_s[t] * y[r]);
          part[r] = to_f32(vv_s[t * LDO + 16 * j + tq]) * y[r];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float x = part[r];
          x += __shfl_xor(x, 8);
          x += __shfl_xor(x, 4);
          x += __shfl_xor(x, 2);
          x += __shfl_xor(x, 1);
          if (tq == 0) atomicAdd(&dbet_s[t0 + 4 * q + r], x);
        }
      }
      __syncthreads();
      if constexpr (BFV) {
        // One 32x32x16 bf16 step per 16 values of the slice; fp32 operands
        // split (mfma_tiles.h).
        auto vstep = [&](const int c0) {
        if (own) {
          const SplitBf8 bs = col_split_bf8(s_s, LS, 32 * kt + li, c0);
          const SplitBf8 bds = col_split_bf8(ds_s, LS, 32 * kt + li, c0);
#pragma unroll
          for (int m = 0; m < NTW; ++m) {
            const int row = 32 * tile_rt(m) + li;
            if (has_q) mma_exact_split(dq[m], row_bf8(do_s, LDO, row, c0), bs);
            mma_split(dka[m], col_split_bf8(d_s, LT, row, c0), bds);
            mma_split(dkw[m], col_split_bf8(y_s, LT, row, c0), bs);
          }
        }
        const SplitBf8 bu = col_split_bf8(d_s, LT, 32 * ru + li, c0);
        if (grp_p) {
          if (has_q) mma_exact_split(dp, row_bf8(do_s, LDO, 32 * rr + li, c0), bu);
        } else {
          mma_split(dp, col_split_bf8(dd_s, LT, 32 * rr + li, c0), bu);
        }
        };
        if constexpr (VS == 16) {
          vstep(8 * hh);
        } else {
          // not unrolled: two steps' split operands live at once spill at 128 keys
#pragma unroll 1
          for (int ss = 0; ss < VS / 16; ++ss) vstep(16 * ss + 8 * hh);
        }
      } else {
#pragma unroll
      for (int g = 0; g < VS / 8; ++g) {
        const int c0 = 8 * g + 4 * hh;
        if (own) {
          const f32x4 bs = ld_x(s_s, LS, 32 * kt + li, c0), bds = ld_x(ds_s, LS, 32 * kt + li, c0);
#pragma unroll
          for (int m = 0; m < NTW; ++m) {
            const int row = 32 * tile_rt(m) + li;
            if (has_q) mma8(dq[m], ld_c(do_s, LDO, row, c0), bs);
            mma8(dka[m], ld_x(d_s, LT, row, c0), bds);
            mma8(dkw[m], ld_x(y_s, LT, row, c0), bs);
          }
        }
        const f32x4 bu = ld_x(d_s, LT, 32 * ru + li, c0);
        if (grp_p) {
          if (has_q) mma8(dp, ld_c(do_s, LDO, 32 * rr + li, c0), bu);
        } else {
          mma8(dp, ld_x(dd_s, LT, 32 * rr + li, c0), bu);
        }
      }
      }
      __syncthreads();
      if (PREFETCH && sl + 1 < nsl) {
        stash();
        __syncthreads();
      }
    }
  }

  // ---- value-axis terms: scale rows, gate gradients, merge the Y term into dKn.
  if (own) {
    const int k = 32 * kt + li;
    float rk_total = 0.f;
#pragma unroll
    for (int m = 0; m < NTW; ++m) {
      const int rt = tile_rt(m);
      float pq[16], pk[16], pw[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = 32 * rt + acc_row(r, hh);
        const float eg = eg_s[t], ek = ek_s[t];
        const float kv = kr(t, k);
        if (has_q) {
          dq[m][r] *= eg;
          pq[r] = qr(t, k) * dq[m][r];
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
        const float eg = eg_s[t];
        atomicAdd(&dgam_s[t], sq - sk + bet_s[t] * eg * sw);
        atomicAdd(&dbet_s[t], eg * sw);
        rk_total += sk;
      }
    }
    rk_total = sum64(rk_total);
    if (lane == 0) atomicAdd(&dgam_s[R - 1], rk_total);
  }

  // ---- P (waves 0-3) and KK (waves 4-7) on the R x R tile: contraction over all keys.
  f32x16 pk2 = {};
  if (!grp_p || has_q) {
    if (std::is_same<E, bf16_t>::value) {
      // bf16 MFMA: the rounded rows are exact in bf16 (32x32x16, lane l holds
      // row l%32, columns 16 g + 8 (l/32) .. +7).
#pragma unroll 4
      for (int g = 0; g < KM / 16; ++g) {
        const int c0 = 16 * g + 8 * hh;
        bf16x8 a, bk;
        if (XR) {
          a = *reinterpret_cast<const bf16x8*>((grp_p ? xqb : xkb) + (32 * rr + li) * LX + c0);
          bk = *reinterpret_cast<const bf16x8*>(xkb + (32 * ru + li) * LX + c0);
        } else {
          a = pack8((grp_p ? xq_s : xk_s) + (32 * rr + li) * LX + c0);
          bk = pack8(xk_s + (32 * ru + li) * LX + c0);
        }
        pk2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bk, pk2, 0, 0, 0);
      }
    } else {
#pragma unroll 4
      for (int g = 0; g < KM / 8; ++g) {
        const int c0 = 8 * g + 4 * hh;
        mma8(pk2, ld_c(grp_p ? xq_s : xk_s, LX, 32 * rr + li, c0), ld_c(xk_s, LX, 32 * ru + li, c0));
      }
    }
  }
  {
    const int u = 32 * ru + li;
    if (grp_p) {
      // ---- dP: gate gradients and dQK.
      float prow[16], pcol = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = 32 * rr + acc_row(r, hh);
        const bool live = u <= t;
        const float e = live ? __expf(gam_s[t] - gam_s[u]) : 0.f;
        const float dpv = (has_q && live) ? dp[r] : 0.f;
        const float g = dpv * e * pk2[r];
        prow[r] = g;
        pcol += g;
        dqk[t * LT + u] = dpv * e;
      }
      const float srow = tile_row_sum(prow, lane);
      if ((lane & 1) == 0) atomicAdd(&dgam_s[32 * rr + acc_row(sum_index(lane), hh)], srow);
      pcol += __shfl_xor(pcol, 32);
      if (hh == 0) atomicAdd(&dgam_s[u], -pcol);
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) xm[(32 * rr + acc_row(r, hh)) * LT + u] = dp[r];
    }
    __syncthreads();
    // ---- dA = -(T^T X), strictly lower (waves 4-7): b, gate and dKK.
    f32x16 da = {};
    if (!grp_p && BFV) {
#pragma unroll
      for (int g = 0; g < R / 16; ++g) {
        const int c0 = 16 * g + 8 * hh;
        mma_split(da, col_split_bf8(tm, LT, 32 * rr + li, c0), col_split_bf8(xm, LT, 32 * ru + li, c0));
      }
    } else if (!grp_p) {
#pragma unroll
      for (int g = 0; g < R / 8; ++g) {
        const int c0 = 8 * g + 4 * hh;
        mma8(da, ld_x(tm, LT, 32 * rr + li, c0), ld_x(xm, LT, 32 * ru + li, c0));
      }
    }
    __syncthreads();  // xm is read by every wave before dKK overwrites it
    if (!grp_p) {
      float rb[16], rg[16], gcol = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = 32 * rr + acc_row(r, hh);
        const bool live = u < t;  // e^{G_t-G_u} may overflow above the diagonal
        const float dav = live ? -da[r] : 0.f;
        const float e = live ? __expf(gam_s[t] - gam_s[u]) : 0.f;
        const float ekk = e * pk2[r];
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

  // ---- position-axis terms, then the normalisation backward.
  // Exact x/|x| at this lane's tile elements (the raw rows when XR).
  float xe[NTW][16], qe[NTW][16];
  if (own) {
    const int k = 32 * kt + li;
    if constexpr (BFV) {
    // bf16: Kn, Qn rows exact, dQK and dKK + dKK^T split.
#pragma unroll 2
    for (int g = 0; g < R / 16; ++g) {
      const int c0 = 16 * g + 8 * hh;
      bf16x8 bk, bq;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        bk[e] = (__bf16)kr(c0 + e, k);
        bq[e] = (__bf16)qr(c0 + e, k);
      }
#pragma unroll
      for (int m = 0; m < NTW; ++m) {
        const int row = 32 * tile_rt(m) + li;
        if (has_q) {
          mma_split_exact(dq[m], row_split_bf8(dqk, LT, row, c0), bk);
          mma_split_exact(dka[m], col_split_bf8(dqk, LT, row, c0), bq);
        }
        float kk[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) kk[e] = dkk[row * LT + c0 + e] + dkk[(c0 + e) * LT + row];
        mma_split_exact(dka[m], split_bf8(kk), bk);
      }
    }
    } else {
#pragma unroll 2
    for (int g = 0; g < R / 8; ++g) {
      const int c0 = 8 * g + 4 * hh;
      const f32x4 bk = f32x4{kr(c0, k), kr(c0 + 1, k), kr(c0 + 2, k), kr(c0 + 3, k)};
      const f32x4 bq = f32x4{qr(c0, k), qr(c0 + 1, k), qr(c0 + 2, k), qr(c0 + 3, k)};
#pragma unroll
      for (int m = 0; m < NTW; ++m) {
        const int row = 32 * tile_rt(m) + li;
        if (has_q) {
          mma8(dq[m], ld_c(dqk, LT, row, c0), bk);
          mma8(dka[m], ld_x(dqk, LT, row, c0), bq);
        }
        mma8(dka[m], ld_c(dkk, LT, row, c0) + ld_x(dkk, LT, row, c0), bk);
      }
    }
    }
    if (XR) {
      const bool kin = k < K;
#pragma unroll
      for (int m = 0; m < NTW; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int tok = tok_s[32 * tile_rt(m) + acc_row(r, hh)];
          const bool ok = tok >= 0 && kin;
          const int tt = ok ? tok : 0, kk = ok ? k : 0;
          xe[m][r] = op_load<E>(p.k, b, h, tt, kk);
          qe[m][r] = op_load<E>(qsrc, b, h, tt, kk);
        }
#pragma unroll
      for (int m = 0; m < NTW; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = 32 * tile_rt(m) + acc_row(r, hh);
          const bool ok = tok_s[t] >= 0 && kin;
          xe[m][r] = ok ? xe[m][r] * krd_s[t] : 0.f;
          qe[m][r] = (ok && has_q) ? qe[m][r] * qrd_s[t] : 0.f;
        }
    } else {
#pragma unroll
      for (int m = 0; m < NTW; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = 32 * tile_rt(m) + acc_row(r, hh);
          xe[m][r] = xk_s[t * LX + k];
          qe[m][r] = xq_s[t * LX + k];
        }
    }
    // part 1: x/|x| . dX per row
#pragma unroll
    for (int m = 0; m < NTW; ++m) {
      float ck[16], cq[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        ck[r] = xe[m][r] * dka[m][r];
        cq[r] = qe[m][r] * dq[m][r];
      }
      const float sk = tile_row_sum(ck, lane);
      const float sq = has_q ? tile_row_sum(cq, lane) : 0.f;
      if ((lane & 1) == 0) {
        const int t = 32 * tile_rt(m) + acc_row(sum_index(lane), hh);
        atomicAdd(&kdot_s[t], sk);
        if (has_q) atomicAdd(&qdot_s[t], sq);
      }
    }
  }

  ddot = sum64(ddot);
  if (lane == 0) atomicAdd(&red_s[0], ddot);
  __syncthreads();
  if (tid == 0) dgam_s[R - 1] += __expf(gc) * red_s[0];

  // ---- part 2: dX = (g - x^ (x^ . g)) / |x|.
  if (own) {
    const int k = 32 * kt + li;
    E* dqo = gr.dq.ptr && p.q.ptr ? reinterpret_cast<E*>(gr.dq.ptr) + op_base(gr.dq, b, h) : nullptr;
    E* dko = reinterpret_cast<E*>(gr.dk.ptr) + op_base(gr.dk, b, h);
    if (k < K) {
#pragma unroll
      for (int m = 0; m < NTW; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = 32 * tile_rt(m) + acc_row(r, hh);
          const int tok = tok_s[t];
          if (tok < 0) continue;
          dko[(int64_t)tok * gr.dk.st + k] =
              from_f32<E>((knrm_s[t] > 1e-6f ? dka[m][r] - xe[m][r] * kdot_s[t] : dka[m][r]) * krd_s[t]);
          if (has_q) {
            dqo[(int64_t)tok * gr.dq.st + k] =
                from_f32<E>((qnrm_s[t] > 1e-6f ? dq[m][r] - qe[m][r] * qdot_s[t] : dq[m][r]) * qrd_s[t]);
          } else if (dqo) {
            dqo[(int64_t)tok * gr.dq.st + k] = from_f32<E>(0.f);
          }
        }
    }
  }
  __syncthreads();
  static_assert(R == 64, "one chunk row per lane of wave 0");
  if (wave == 0) {
    // dg_t = sum_{u >= t} dgam_u: a suffix sum across the wave's lanes
    float acc = dgam_s[lane];
#pragma unroll
    for (int off = 1; off < R; off <<= 1) {
      const float o = __shfl_down(acc, off, 64);
      if (lane + off < R) acc += o;
    }
    const int tok = tok_s[lane];
    if (tok >= 0) {
      reinterpret_cast<float*>(gr.dg.ptr)[op_base(gr.dg, b, h) + (int64_t)tok * gr.dg.st] = acc;
      reinterpret_cast<float*>(gr.dbeta.ptr)[op_base(gr.dbeta, b, h) + (int64_t)tok * gr.dbeta.st] = dbet_s[lane];
    }
  }
}

template <typename E, int KM>
size_t chunk_bwd_mfma_lds() {
  return ChunkBwdLayout<E, KM>::BYTES;
}

template <typename E, int KM>
int launch_chunk_bwd_mfma(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, const gpa_gdn_grads& gr, int nch,
                          hipStream_t st) {
  const size_t lds = ChunkBwdLayout<E, KM>::BYTES;
  if (lds > 65536) {
    const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(gdn_chunk_bwd_mfma<E, KM>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (err != hipSuccess) return fail(GPA_HIP_EHIP, "hipFuncSetAttribute(max dynamic LDS) failed");
  }
  hipLaunchKernelGGL((gdn_chunk_bwd_mfma<E, KM>), dim3(nch, p.batch * p.heads), dim3(CB_NT), lds, st, p, sv, gr, nch);
  return GPA_HIP_OK;
}

#define GPA_CHUNK_BWD_MFMA(E, KM)                                                                              \
  template size_t chunk_bwd_mfma_lds<E, KM>();                                                                  \
  template int launch_chunk_bwd_mfma<E, KM>(const gpa_gdn_problem&, const gpa_gdn_saved&, const gpa_gdn_grads&, \
                                            int, hipStream_t);
GPA_CHUNK_BWD_MFMA(float, 64)
GPA_CHUNK_BWD_MFMA(float, 128)
GPA_CHUNK_BWD_MFMA(bf16_t, 64)
GPA_CHUNK_BWD_MFMA(bf16_t, 128)
GPA_CHUNK_BWD_MFMA(bf16_t, 256)
#undef GPA_CHUNK_BWD_MFMA

}  // namespace gpa
