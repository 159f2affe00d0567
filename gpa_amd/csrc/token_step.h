// The one-token GDN step of one column block of one stream's state (the
// inference decode of the chunk model at T = 1): reference src/gpa/ops.py:29-42
// (gdn_update) then :45-46 (memory_read).  Shared by the one-token step
// kernels and the kernel that runs a level's inner step beside its one-token
// level write.
#pragma once

#include "glue_rows.h"

namespace gpa {
namespace {

constexpr int SNT = 256;   // threads per workgroup

// The row classes (K <= 16 NI): a workgroup owns SC columns of one stream's
// state, thread t columns 4 (t % CQ) .. +3 of rows t / CQ + RG i, i < NR.
// K <= 128 takes 64-column blocks (16 column quads x 16 row groups); the
// 256-row class takes 32-column blocks (8 x 32), so that a thread holds 8
// rows as at K = 128, not 16: half the registers, twice the workgroups
// resident per compute unit.
template <int NI>
struct TokenShape {
  static constexpr int SC = NI == 16 ? 32 : 64;
  static constexpr int CQ = SC / 4, RG = SNT / CQ, NR = 16 * NI / RG;
};
__host__ __device__ constexpr int token_cols(int ni) { return ni == 16 ? 32 : 64; }

// Sum of the row groups that share a wave's column quad (lanes c, c + CQ,
// ...), then of the four waves through LDS; every thread returns the total
// of its quad.
template <int CQ>
__device__ __forceinline__ float4 column_sums(float4 x, float4 (*part)[CQ], int wave, int rg, int c4) {
#pragma unroll
  for (int m = CQ; m < 64; m *= 2) {
    x.x += __shfl_xor(x.x, m, 64);
    x.y += __shfl_xor(x.y, m, 64);
    x.z += __shfl_xor(x.z, m, 64);
    x.w += __shfl_xor(x.w, m, 64);
  }
  if ((rg & (64 / CQ - 1)) == 0) part[wave][c4] = x;
  lds_barrier();
  float4 s = part[0][c4];
#pragma unroll
  for (int w = 1; w < 4; ++w) {
    const float4 y = part[w][c4];
    s.x += y.x;
    s.y += y.y;
    s.z += y.z;
    s.w += y.w;
  }
  return s;
}

// Workgroup wg of one problem (one SC-column block of one stream).
template <int NI>
struct TokenLds {
  float kh[16 * NI], qh[16 * NI];
  float norms[2][4];
  float4 part[2][4][TokenShape<NI>::CQ];
  float kraw[16 * NI];             // the key as given (slot products in the step)
  float vsl[TokenShape<NI>::SC];   // this block's slot values
  float gates[2];                  // g_in, b_in
};

// The step's value and gates formed in the step (gpa_token_slot): slot
// columns SC cb .. of stream (b, h), SNT / SC threads per column over 8-wide
// key chunks of C's row (16-byte loads), summed by shuffles and rounded to
// bf16; wave 0 forms the gate inputs round(unit(k) W_g) and their
// nonlinearities (gate_values), written out by the stream's first block.
// slot_loads issues the loads of C and W_g before the state's, so that the
// products wait for them alone; slot_gates then runs once the rounded unit
// key kh and the key kraw are in LDS.
template <int NI>
struct SlotRegs {
  static constexpr int TPC = SNT / TokenShape<NI>::SC, CR = 16 * NI / (8 * TPC), GR = 16 * NI / 64;
  uint4 c[CR];   // this thread's 8-wide chunks of its C row
  uint2 w[GR];   // W_g rows d = lane + 64 i (wave 0)
};

template <int NI>
__device__ __forceinline__ void slot_loads(const gpa_token_slot& ts, int h, int cb, int t, int K, int V,
                                           SlotRegs<NI>& R) {
  constexpr int SC = TokenShape<NI>::SC, TPC = SlotRegs<NI>::TPC;
  const int c = t / TPC, part = t % TPC, m = SC * cb + c;
  const bf16_t* cr = reinterpret_cast<const bf16_t*>(ts.center) + ((int64_t)h * V + (m < V ? m : V - 1)) * K;
#pragma unroll
  for (int i = 0; i < SlotRegs<NI>::CR; ++i) {
    const int d0 = 8 * (part + TPC * i);
    R.c[i] = *reinterpret_cast<const uint4*>(cr + (d0 < K ? d0 : 0));
  }
  if (t < 64) {
    const bf16_t* gw = reinterpret_cast<const bf16_t*>(ts.gate_w) + (int64_t)h * K * 4;
#pragma unroll
    for (int i = 0; i < SlotRegs<NI>::GR; ++i) {
      const int d = t + 64 * i;
      R.w[i] = *reinterpret_cast<const uint2*>(gw + 4 * (d < K ? d : 0));
    }
  }
}

template <int NI>
__device__ __forceinline__ void slot_gates(const gpa_token_slot& ts, const SlotRegs<NI>& R, int b, int h, int H,
                                           int cb, int t, int K, int V, TokenLds<NI>& L) {
  constexpr int SC = TokenShape<NI>::SC, TPC = SlotRegs<NI>::TPC;
  const int c = t / TPC, part = t % TPC, m = SC * cb + c, lane = t & 63;
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < SlotRegs<NI>::CR; ++i) {
    const int d0 = 8 * (part + TPC * i);
    if (d0 < K) {
      const uint32_t ww[4] = {R.c[i].x, R.c[i].y, R.c[i].z, R.c[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc += L.kraw[d0 + 2 * e] * __uint_as_float(ww[e] << 16);
        acc += L.kraw[d0 + 2 * e + 1] * __uint_as_float(ww[e] & 0xffff0000u);
      }
    }
  }
#pragma unroll
  for (int o = 1; o < TPC; o *= 2) acc += __shfl_xor(acc, o, 64);
  if (part == 0 && m < V) {
    const bf16_t sv = from_f32<bf16_t>(acc);
    L.vsl[c] = to_f32(sv);
    reinterpret_cast<bf16_t*>(ts.slot.ptr)[op_base(ts.slot, b, h) + m] = sv;
  }
  if (t < 64) {
    float g4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < SlotRegs<NI>::GR; ++i) {
      const int d = lane + 64 * i;
      if (d < K) {
        const float u = L.kh[d];
        g4[0] += u * __uint_as_float(R.w[i].x << 16);
        g4[1] += u * __uint_as_float(R.w[i].x & 0xffff0000u);
        g4[2] += u * __uint_as_float(R.w[i].y << 16);
        g4[3] += u * __uint_as_float(R.w[i].y & 0xffff0000u);
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) g4[q] = round_as<bf16_t>(sum64(g4[q]));
    if (lane == 0) {
      float v[4];
      gate_values(ts.gates, h, g4, v);
      L.gates[0] = v[0];
      L.gates[1] = v[1];
      if (cb == 0) {
        const int64_t i = (int64_t)b * H + h;
        ts.gates.g_in[i] = v[0];
        ts.gates.b_in[i] = v[1];
        ts.gates.g_out[i] = v[2];
        ts.gates.b_out[i] = v[3];
      }
    }
  }
}

// t: the thread's index in its 256-thread unit; every thread of the
// workgroup reaches the same barriers (the units of a workgroup run one
// problem, so `update` and `has_q` agree).  SLOT: the value, decay and
// strength come from token_slot_gates (an update; bf16 activations).
template <typename E, int NI, bool SLOT = false>
__device__ __forceinline__ void token_run(const gpa_gdn_problem& p, float* fin, const gpa_operand& out, int wg, int t,
                                          TokenLds<NI>& L, const gpa_token_slot& ts) {
  constexpr int SC = TokenShape<NI>::SC, CQ = TokenShape<NI>::CQ, RG = TokenShape<NI>::RG;
  constexpr int NR = TokenShape<NI>::NR;
  float* const kh = L.kh;
  float* const qh = L.qh;
  float (*const norms)[4] = L.norms;
  float4 (*const part)[4][CQ] = L.part;
  const int ncb = (p.vdim + SC - 1) / SC;
  const int s = wg / ncb, cb = wg - s * ncb;
  const int b = s / p.heads, h = s - b * p.heads;
  const int lane = t & 63, wave = t >> 6;
  const int c4 = t % CQ, rg = t / CQ;
  const int K = p.kdim, V = p.vdim;
  const int col = SC * cb + 4 * c4;
  const bool cok = col < V;  // V % 4 == 0: a quad is all inside or all outside
  const int cc = cok ? col : 0;
  const bool update = p.k.ptr != nullptr, has_q = p.q.ptr != nullptr;

  // Every load first, at clamped addresses, the small ones before the state
  // (the norms and slot products wait for them alone); masks afterwards.
  const int tk = t < K ? t : 0;
  float xk = 0.f, xq = 0.f, vv[4] = {0.f, 0.f, 0.f, 0.f}, g = 0.f, beta = 0.f;
  if (update) {
    xk = op_load<E>(p.k, b, h, 0, tk);
    if (!SLOT) {
#pragma unroll
      for (int j = 0; j < 4; ++j) vv[j] = op_load<E>(p.v, b, h, 0, cc + j);
      g = scalar_load(p.g, b, h, 0);
      beta = scalar_load(p.beta, b, h, 0);
    }
  }
  if (has_q) xq = op_load<E>(p.q, b, h, 0, tk);
  SlotRegs<NI> sr;
  if constexpr (SLOT) slot_loads<NI>(ts, h, cb, t, K, V, sr);
  const float* s0 = p.s0 ? p.s0 + (int64_t)b * p.s0_sb + (int64_t)h * p.s0_sh : nullptr;
  float4 st[NR];
  if (s0) {
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const int row = rg + RG * i;
      st[i] = *reinterpret_cast<const float4*>(s0 + (int64_t)(row < K ? row : 0) * V + cc);
    }
  } else {
#pragma unroll
    for (int i = 0; i < NR; ++i) st[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  xk = t < K ? xk : 0.f;
  xq = t < K ? xq : 0.f;
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const bool ok = s0 && cok && rg + RG * i < K;
    st[i] = ok ? st[i] : make_float4(0.f, 0.f, 0.f, 0.f);
  }

  // u(k) and u(q): x / max(||x||, 1e-6), rounded to the activation type
  // (reference ops.py:14-17).
  const float sk = sum64(xk * xk), sq = sum64(xq * xq);
  if (lane == 0) {
    norms[0][wave] = sk;
    norms[1][wave] = sq;
  }
  lds_barrier();
  const float nk = fmaxf(sqrtf(norms[0][0] + norms[0][1] + norms[0][2] + norms[0][3]), 1e-6f);
  const float nq = fmaxf(sqrtf(norms[1][0] + norms[1][1] + norms[1][2] + norms[1][3]), 1e-6f);
  if (t < 16 * NI) {
    kh[t] = t < K ? round_as<E>(xk / nk) : 0.f;
    qh[t] = t < K ? round_as<E>(xq / nq) : 0.f;
    if (SLOT) L.kraw[t] = xk;
  }
  lds_barrier();
  if constexpr (SLOT) {
    slot_gates<NI>(ts, sr, b, h, p.heads, cb, t, K, V, L);
    lds_barrier();
#pragma unroll
    for (int j = 0; j < 4; ++j) vv[j] = cok ? L.vsl[4 * c4 + j] : 0.f;
    g = L.gates[0];
    beta = L.gates[1];
  }

  if (update) {
    // scaled = exp(g) S; predicted = u(k)^T scaled; S' = scaled + beta (u(k) (v - predicted)^T)
    const float a = expf(g);
    float4 pk = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const float kr = kh[rg + RG * i];
      st[i].x *= a;
      st[i].y *= a;
      st[i].z *= a;
      st[i].w *= a;
      pk.x += kr * st[i].x;
      pk.y += kr * st[i].y;
      pk.z += kr * st[i].z;
      pk.w += kr * st[i].w;
    }
    const float4 pred = column_sums<CQ>(pk, part[0], wave, rg, c4);
    const float r0 = vv[0] - pred.x, r1 = vv[1] - pred.y, r2 = vv[2] - pred.z, r3 = vv[3] - pred.w;
    float* dst = fin + (int64_t)s * K * V;
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const int row = rg + RG * i;
      const float kr = kh[row];
      st[i].x += beta * (kr * r0);
      st[i].y += beta * (kr * r1);
      st[i].z += beta * (kr * r2);
      st[i].w += beta * (kr * r3);
      if (cok && row < K) *reinterpret_cast<float4*>(dst + (int64_t)row * V + col) = st[i];
    }
  }

  if (has_q) {
    float4 po = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const float qr = qh[rg + RG * i];
      po.x += qr * st[i].x;
      po.y += qr * st[i].y;
      po.z += qr * st[i].z;
      po.w += qr * st[i].w;
    }
    const float4 o = column_sums<CQ>(po, part[1], wave, rg, c4);
    if (t < CQ && cok) {
      E* op = reinterpret_cast<E*>(out.ptr) + op_base(out, b, h) + col;
      op[0] = from_f32<E>(o.x);
      op[1] = from_f32<E>(o.y);
      op[2] = from_f32<E>(o.z);
      op[3] = from_f32<E>(o.w);
    }
  }
}

int token_rows(const gpa_gdn_problem& p) { return p.kdim <= 64 ? 4 : (p.kdim <= 128 ? 8 : 16); }
int64_t token_workgroups(const gpa_gdn_problem& p) {
  const int sc = token_cols(token_rows(p));
  return (int64_t)p.batch * p.heads * ((p.vdim + sc - 1) / sc);
}

bool aligned16(const void* x) { return ((uintptr_t)x & 15) == 0; }

int check_token(const gpa_gdn_problem* problem, const float* final_state, const gpa_operand& out) {
  if (!problem) return fail(GPA_HIP_EINVAL, "token step: null problem");
  const gpa_gdn_problem& p = *problem;
  if (p.tokens != 1) return fail(GPA_HIP_EINVAL, "token step: needs tokens == 1");
  if (p.batch < 1 || p.heads < 1 || p.kdim < 1 || p.vdim < 1) return fail(GPA_HIP_EINVAL, "token step: empty shape");
  if (p.kdim > 256 || p.vdim > 256) return fail(GPA_HIP_EUNSUPPORTED, "token step: widths above 256");
  if (p.vdim % 4) return fail(GPA_HIP_EUNSUPPORTED, "token step: V must be a multiple of 4");
  if (p.dtype != GPA_DTYPE_F32 && p.dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "token step: dtype");
  const bool update = p.k.ptr != nullptr;
  if (update && (!p.v.ptr || !p.g.ptr || !p.beta.ptr || !final_state))
    return fail(GPA_HIP_EINVAL, "token step: an update needs v, g, beta and final");
  if (!update && (!p.q.ptr || !p.s0)) return fail(GPA_HIP_EINVAL, "token step: a read needs q and s0");
  if (p.q.ptr && !out.ptr) return fail(GPA_HIP_EINVAL, "token step: a query needs out");
  if (p.s0 && (!aligned16(p.s0) || p.s0_sb % 4 || p.s0_sh % 4))
    return fail(GPA_HIP_EINVAL, "token step: s0 must be 16-byte aligned with strides a multiple of 4");
  if (final_state && !aligned16(final_state)) return fail(GPA_HIP_EINVAL, "token step: final must be 16-byte aligned");
  if (token_workgroups(p) > INT32_MAX / 2) return fail(GPA_HIP_EINVAL, "token step: too many streams");
  return GPA_HIP_OK;
}

}  // namespace
}  // namespace gpa
