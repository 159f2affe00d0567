// The read of the chunked GDN scan and the chunk-local part of its gradient
// on bf16 MFMA (gfx950 v_mfma_f32_32x32x16_bf16), one block per (chunk,
// stream), 4 waves.  Within a chunk of positions t, u:
//   P   = causal e^{G_t-G_u} Qn Kn^T
//   O   = diag(e^G) Qn S_n + P D                 (gdn_out_mfma)
//   dd0 = P^T dO,   o = diag(e^G) dO             (gdn_dd0_mfma, value-major)
// Qn and Kn are exact in bf16 (the model rounds them to the activation type)
// and saved as bf16 rows (qk_rows_bf16); the fp32 operands S_n, D and P are
// split into bf16 hi + lo and multiplied as hi*hi + hi*lo + lo*hi, with fp32
// accumulation.  Every global operand is read as contiguous bytes per lane
// straight into MFMA fragments (16 for a bf16 row, 32 for fp32): Qn and Kn
// rows are position-major, and the chunk-start states and D are value-major,
// so a lane's eight contraction indices of one value column are contiguous.
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


// Eight contiguous floats split into bf16 hi and lo = bf16(x - hi).
__device__ __forceinline__ void frag_split(const float* x, bf16x8& hi, bf16x8& lo) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(x), c = *reinterpret_cast<const f32x4*>(x + 4);
  const float v[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
  split8(v, hi, lo);
}

// Eight contiguous floats kept raw: a group's loads are all issued before the
// first conversion, so that the wave waits once per group, not per load.
struct Raw8 {
  f32x4 a, b;
};
__device__ __forceinline__ Raw8 ld_raw8(const float* x) {
  return Raw8{*reinterpret_cast<const f32x4*>(x), *reinterpret_cast<const f32x4*>(x + 4)};
}
__device__ __forceinline__ void split_of(const Raw8& r, bf16x8& hi, bf16x8& lo) {
  const float v[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
  split8(v, hi, lo);
}
// Fragments loaded per group (fewer with 256 keys, whose Qn fragments
// already hold 64 registers).
template <int KM>
constexpr int lgroup() {
  return KM > 128 ? 4 : 8;
}

// Eight contiguous bf16 of a saved Qn / Kn row (bf16 rows: qk_rows_bf16).
__device__ __forceinline__ bf16x8 ld_bf8(const bf16_t* x) {
  const uint4 w = *reinterpret_cast<const uint4*>(x);
  bf16x8 r;
  __builtin_memcpy(&r, &w, 16);
  return r;
}

// The (rt, ct) 32x32 tile of P = causal e^{G_t-G_u} Qn Kn^T, with qa the Qn
// fragments of row tile rt (K16 k steps) and krow the chunk's Kn row
// fragments (the state kernels' krow: fragment (ct, ks), lane l holds
// Kn[32 ct + l%32][16 ks + 8 (l/32) + e]).  Lane l ends with column
// u = 32 ct + l%32 and rows t = 32 rt + acc_row(r, l/32).
template <int KM>
__device__ __forceinline__ f32x16 p_tile(const bf16x8 (&qa)[KM / 16], const bf16_t* krow, int K16, int rt, int ct,
                                         int l, const float* gam_s) {
  const int li = l & 31, hh = l >> 5;
  f32x16 acc = {};
  const bf16_t* kf = krow + ((int64_t)ct * K16 * 64 + l) * 8;
#pragma unroll
  for (int k0 = 0; k0 < KM / 16; k0 += lgroup<KM>()) {
    bf16x8 kb[lgroup<KM>()];
#pragma unroll
    for (int j = 0; j < lgroup<KM>() && k0 + j < KM / 16; ++j) kb[j] = ld_bf8(kf + 512 * (k0 + j < K16 ? k0 + j : 0));
#pragma unroll
    for (int j = 0; j < lgroup<KM>() && k0 + j < KM / 16; ++j)
      if (k0 + j < K16) acc = mfma_bf16(qa[k0 + j], kb[j], acc);
  }
  const int u = 32 * ct + li;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int t = 32 * rt + acc_row(r, hh);
    acc[r] = u <= t ? __expf(gam_s[t] - gam_s[u]) * acc[r] : 0.f;
  }
  return acc;
}

template <int KM>
__device__ __forceinline__ void load_q(bf16x8 (&qa)[KM / 16], const bf16_t* qn, int K16, int K, int rt, int l) {
  const bf16_t* qrow = qn + (32 * rt + (l & 31)) * K + 8 * (l >> 5);
#pragma unroll
  for (int k0 = 0; k0 < KM / 16; k0 += lgroup<KM>()) {
    bf16x8 raw[lgroup<KM>()];
#pragma unroll
    for (int j = 0; j < lgroup<KM>() && k0 + j < KM / 16; ++j) raw[j] = ld_bf8(qrow + 16 * (k0 + j < K16 ? k0 + j : 0));
#pragma unroll
    for (int j = 0; j < lgroup<KM>() && k0 + j < KM / 16; ++j) qa[k0 + j] = k0 + j < K16 ? raw[j] : bf16x8{};
  }
}
// The saved bf16 rows (qk_rows_bf16 holds wherever these kernels run).
__device__ __forceinline__ const bf16_t* rows16(const float* base, int64_t off) {
  return reinterpret_cast<const bf16_t*>(base) + off;
}
// Chunk n of stream s in the Kn row fragments.
__device__ __forceinline__ const bf16_t* krow_of(const gpa_gdn_saved& sv, int s, int n, int nch, int K) {
  return reinterpret_cast<const bf16_t*>(sv.krow) + ((int64_t)s * nch + n) * frag_row_elems(K, 8);
}

}  // namespace

// O = diag(e^G) Qn S_n + P D for one (chunk n, stream s); V <= 256.
template <int KM>
__global__ __launch_bounds__(ONT, 2) void gdn_out_mfma(gpa_gdn_problem p, gpa_gdn_saved sv, gpa_operand out, int nch) {
  __shared__ __align__(16) __bf16 ph[R * PLD], pl[R * PLD];  // P hi / lo, [t][u]
  __shared__ float gam_s[R];
  const int n = blockIdx.x, s = blockIdx.y, b = s / p.heads, h = s % p.heads;
  const int K = p.kdim, V = p.vdim, K16 = K / 16, tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int li = l & 31, hh = l >> 5, rt = w & 1;
  if (tid < R) gam_s[tid] = sv.gam[rows_off(s, n, nch, 0, 1) + tid];
  bf16x8 qa[KM / 16];
  load_q<KM>(qa, rows16(sv.qn, rows_off(s, n, nch, 0, K)), K16, K, rt, l);
  __syncthreads();
  {
    const f32x16 pt = p_tile<KM>(qa, krow_of(sv, s, n, nch, K), K16, rt, w >> 1, l, gam_s);
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
    const float* drow = dl + (int64_t)vc * R + 8 * hh;
#pragma unroll
    for (int k0 = 0; k0 < KM / 16; k0 += lgroup<KM>()) {
      Raw8 raw[lgroup<KM>()];
#pragma unroll
      for (int j = 0; j < lgroup<KM>() && k0 + j < KM / 16; ++j) raw[j] = ld_raw8(srow + 16 * (k0 + j < K16 ? k0 + j : 0));
#pragma unroll
      for (int j = 0; j < lgroup<KM>() && k0 + j < KM / 16; ++j)
        if (k0 + j < K16) {
          bf16x8 bh, bl;
          split_of(raw[j], bh, bl);
          a1 = mfma_bf16(qa[k0 + j], bh, a1);
          a2 = mfma_bf16(qa[k0 + j], bl, a2);
        }
    }
    Raw8 draw[R / 16];
#pragma unroll
    for (int us = 0; us < R / 16; ++us) draw[us] = ld_raw8(drow + 16 * us);
    f32x16 acc = a1 + a2;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] *= __expf(gam_s[32 * rt + acc_row(r, hh)]);
#pragma unroll
    for (int us = 0; us < R / 16; ++us) {
      bf16x8 dh, dlo;
      split_of(draw[us], dh, dlo);
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
// stream s); V <= VM <= 256 (VM = 128 leaves room for more workgroups per CU).
template <int KM, int VM>
__global__ __launch_bounds__(ONT, 2) void gdn_dd0_mfma(gpa_gdn_problem p, gpa_gdn_saved sv, gpa_gdn_grads gr,
                                                     int nch) {
  static_assert(VM <= GPA_OUT_MFMA_MAX_V, "value width");
  __shared__ __align__(16) __bf16 ph[R * PLD], pl[R * PLD];  // P^T hi / lo, [u][t]
  __shared__ __align__(16) __bf16 dot[VM * PLD];  // dO^T, [v][t] (exact)
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
    bf16_t x[8];  // clamped loads first, masks at the stores
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = src[v0 + e < V ? v0 + e : V - 1];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int v = v0 + e;
      if (v < V) reinterpret_cast<bf16_t*>(dot)[v * PLD + t] = tok >= 0 ? x[e] : bf16_t{0};
    }
  }
  bf16x8 qa[KM / 16];
  load_q<KM>(qa, rows16(sv.qn, rows_off(s, n, nch, 0, K)), K16, K, rt, l);
  __syncthreads();
  {
    const f32x16 pt = p_tile<KM>(qa, krow_of(sv, s, n, nch, K), K16, rt, w >> 1, l, gam_s);
    const int u = 32 * (w >> 1) + li;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = 32 * rt + acc_row(r, hh);
      const __bf16 hi = (__bf16)pt[r];
      ph[u * PLD + t] = hi;
      pl[u * PLD + t] = (__bf16)(pt[r] - (float)hi);
    }
  }
  // o = diag(e^G) dO in fragment order (ufrag_idx): thread -> (strip, row
  // tile, group, lane), four consecutive rows of one column; zero past V.
  float* om = gr.o + ufrag_off(s, n, nch, V);
  for (int idx = tid; idx < ((V + 31) / 32) * 512; idx += ONT) {
    const int ln = idx & 63, g = (idx >> 6) & 3, r2 = (idx >> 8) & 1, c = idx >> 9;
    const int v = 32 * c + (ln & 31), t0 = 32 * r2 + 8 * g + 4 * (ln >> 5);
    const bf16_t* x = reinterpret_cast<const bf16_t*>(dot) + (v < V ? v : 0) * PLD + t0;
    *reinterpret_cast<float4*>(om + ufrag_idx(c, r2, g, ln)) =
        v < V ? make_float4(__expf(gam_s[t0]) * to_f32(x[0]), __expf(gam_s[t0 + 1]) * to_f32(x[1]),
                            __expf(gam_s[t0 + 2]) * to_f32(x[2]), __expf(gam_s[t0 + 3]) * to_f32(x[3]))
              : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  __syncthreads();
  float* d0 = gr.dd0 + ufrag_off(s, n, nch, V);
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
#pragma unroll
    for (int g = 0; g < 4; ++g)  // fragment order, zero past V
      *reinterpret_cast<float4*>(d0 + ufrag_idx(vt, ut, g, l)) =
          v < V ? make_float4(acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3])
                : make_float4(0.f, 0.f, 0.f, 0.f);
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
  if (p.vdim <= 128)
    hipLaunchKernelGGL((gdn_dd0_mfma<KM, 128>), dim3(nch, p.batch * p.heads), dim3(ONT), 0, st, p, sv, gr, nch);
  else
    hipLaunchKernelGGL((gdn_dd0_mfma<KM, GPA_OUT_MFMA_MAX_V>), dim3(nch, p.batch * p.heads), dim3(ONT), 0, st, p, sv,
                       gr, nch);
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

// ===========================================================================
// The read of a scan that ran without a query (a late read), and its query
// gradient.  gdn_prep_q normalises the query rows of one (chunk, stream) like
// the scan's own preparation does (x / max(|x|, 1e-6), rounded to the
// activation type) and writes Qn and its fragments; the read itself is
// gdn_out_mfma.  gdn_read_dq_mfma computes the query gradient alone:
//   dQn = diag(e^G) dO S_n^T + (causal e^{G_t-G_u} dO D^T) Kn
//   dq  = (dQn - q^ (q^ . dQn)) / |q|              (q^ = q / |q| unrounded)
// The other gradients of the read (keys, values, gates, states) are those of
// the scan backward with this query and dO, which the caller runs later.
namespace gpa {

template <typename E, int KM, bool MF>
__global__ __launch_bounds__(ONT) void gdn_prep_q(gpa_gdn_problem p, gpa_gdn_saved sv, int nch) {
  const int n = blockIdx.x, s = blockIdx.y, b = s / p.heads, h = s % p.heads;
  const int K = p.kdim, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int NI = KM / 64, NR = R / OWAVES;
  const int64_t chunk_id = (int64_t)s * nch + n;
  __bf16* qcol = MF ? reinterpret_cast<__bf16*>(sv.qcol) + chunk_id * frag_col_elems(K, 8) : nullptr;
  float xq[NR][NI];
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    const int tok = token_at(p, n, wave + OWAVES * j), tt = tok >= 0 ? tok : 0;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int d = lane + 64 * i, dd = d < K ? d : 0;
      xq[j][i] = op_load<E>(p.q, b, h, tt, dd);
    }
  }
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    const int r = wave + OWAVES * j, tok = token_at(p, n, r);
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      xq[j][i] = (tok >= 0 && lane + 64 * i < K) ? xq[j][i] : 0.f;
      sq += xq[j][i] * xq[j][i];
    }
    const float dq = fmaxf(sqrtf(sum64(sq)), 1e-6f);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int d = lane + 64 * i;
      if (d < K) {
        const float yq = round_as<E>(xq[j][i] / dq);
        if (MF) reinterpret_cast<bf16_t*>(sv.qn)[rows_off(s, n, nch, r, K) + d] = from_f32<bf16_t>(yq);
        else sv.qn[rows_off(s, n, nch, r, K) + d] = yq;
        if (MF) {  // Qn^T fragment (d/32, r/16), lane d%32 + 32 ((r/8) % 2), element r % 8
          const int rb = d >> 5, cs = r >> 4, ln = (d & 31) + 32 * ((r >> 3) & 1);
          qcol[((rb * 4 + cs) * 64 + ln) * 8 + (r & 7)] = (__bf16)yq;
        }
      }
    }
  }
}

// LDS of gdn_read_dq_mfma (bf16 elements): S_n^T and D^T of one 64-value
// slice, split (hi, lo), then the masked dO D^T (split) for the Kn product.
template <int KM>
struct ReadDqLayout {
  static constexpr int VSL = 64;
  static constexpr int ST = KM * PLD, DT = R * PLD;
  static constexpr int ST_HI = 0, ST_LO = ST, DT_HI = 2 * ST, DT_LO = DT_HI + DT, END = DT_LO + DT;
  static constexpr size_t BYTES = sizeof(__bf16) * END + sizeof(float) * 4 * R;
};

template <int KM>
__global__ __launch_bounds__(ONT) void gdn_read_dq_mfma(gpa_gdn_problem p, gpa_gdn_saved sv, gpa_operand dout,
                                                         gpa_operand dqo, int nch) {
  using L = ReadDqLayout<KM>;
  constexpr int VSL = L::VSL, NTW = KM >= 64 ? KM / 64 : 1;  // 32x32 dQn tiles per wave
  extern __shared__ __align__(16) unsigned char smem_raw[];
  __bf16* sth = reinterpret_cast<__bf16*>(smem_raw) + L::ST_HI;  // [k][v - v0]
  __bf16* stl = reinterpret_cast<__bf16*>(smem_raw) + L::ST_LO;
  __bf16* dth = reinterpret_cast<__bf16*>(smem_raw) + L::DT_HI;  // [u][v - v0], then dQK [t][u]
  __bf16* dtl = reinterpret_cast<__bf16*>(smem_raw) + L::DT_LO;
  float* gam_s = reinterpret_cast<float*>(reinterpret_cast<__bf16*>(smem_raw) + L::END);
  float* qrd_s = gam_s + R;   // 1 / max(|q_t|, 1e-6)
  float* qnm_s = qrd_s + R;   // |q_t|
  float* qdot_s = qnm_s + R;  // q^ . dQn per row
  const int n = blockIdx.x, s = blockIdx.y, b = s / p.heads, h = s % p.heads;
  const int K = p.kdim, V = p.vdim, tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int li = l & 31, hh = l >> 5, rt = w & 1;
  const int KT = K / 32 > 0 ? (K + 31) / 32 : 1;
  if (tid < R) {
    gam_s[tid] = sv.gam[rows_off(s, n, nch, 0, 1) + tid];
    qdot_s[tid] = 0.f;
  }
  {  // query row norms, 4 threads per row; loads first (clamped), then the sum
    const int row = tid >> 2, part = tid & 3, tok = token_at(p, n, row);
    float xs[KM / 4];
#pragma unroll
    for (int i = 0; i < KM / 4; ++i) {
      const int c = part + 4 * i;
      xs[i] = op_load<bf16_t>(p.q, b, h, tok >= 0 ? tok : 0, c < K ? c : 0);
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < KM / 4; ++i) ss += (tok >= 0 && part + 4 * i < K) ? xs[i] * xs[i] : 0.f;
    ss += __shfl_xor(ss, 1);
    ss += __shfl_xor(ss, 2);
    if (part == 0) {
      const float nq = sqrtf(ss);
      qnm_s[row] = nq;
      qrd_s[row] = 1.f / fmaxf(nq, 1e-6f);
    }
  }
  const float* st = sv.states + state_off(s, n, nch, K, V);
  const float* dl = sv.delta + vc_off(s, n, nch, V);
  // dO rows of this wave's row tile: row t = 32 rt + l%32 (zero for void rows).
  const int tq = 32 * rt + li, tokq = token_at(p, n, tq);
  const bf16_t* dorow = reinterpret_cast<const bf16_t*>(dout.ptr) + op_base(dout, b, h) +
                        (int64_t)(tokq >= 0 ? tokq : 0) * dout.st;
  f32x16 aq[NTW], ap = {};
#pragma unroll
  for (int j = 0; j < NTW; ++j) aq[j] = f32x16{};
  const int pc = w >> 1;  // dO D^T tile (rt, pc)
  for (int v0 = 0; v0 < V; v0 += VSL) {
    __syncthreads();
    // S_n^T slice: thread -> (value v, 4 keys), split into hi / lo; D^T
    // slice: thread -> (value v, 4 positions).  All loads of the thread are
    // issued (at clamped addresses) before the first store.  Lanes take
    // consecutive values, so that a wave's transposed 2-byte stores go to
    // consecutive addresses of one LDS row (lanes along the keys would hit
    // the same few banks).
    constexpr int SN = VSL * (KM / 4) / ONT, DN = VSL * (R / 4) / ONT;
    static_assert(SN * ONT == VSL * (KM / 4) && DN * ONT == VSL * (R / 4), "staging shares");
    float4 xs[SN], xd[DN];
#pragma unroll
    for (int i = 0; i < SN; ++i) {
      const int idx = tid + ONT * i, vl = idx % VSL, k = 4 * (idx / VSL), v = v0 + vl;
      xs[i] = *reinterpret_cast<const float4*>(st + ((v < V && k < K) ? (int64_t)v * K + k : 0));
    }
#pragma unroll
    for (int i = 0; i < DN; ++i) {
      const int idx = tid + ONT * i, vl = idx % VSL, u = 4 * (idx / VSL), v = v0 + vl;
      xd[i] = *reinterpret_cast<const float4*>(dl + (v < V ? (int64_t)v * R + u : 0));
    }
#pragma unroll
    for (int i = 0; i < SN; ++i) {
      const int idx = tid + ONT * i, vl = idx % VSL, k = 4 * (idx / VSL), v = v0 + vl;
      const bool ok = v < V && k < K;
      const float x4[4] = {ok ? xs[i].x : 0.f, ok ? xs[i].y : 0.f, ok ? xs[i].z : 0.f, ok ? xs[i].w : 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const __bf16 hi = (__bf16)x4[e];
        sth[(k + e) * PLD + vl] = hi;
        stl[(k + e) * PLD + vl] = (__bf16)(x4[e] - (float)hi);
      }
    }
#pragma unroll
    for (int i = 0; i < DN; ++i) {
      const int idx = tid + ONT * i, vl = idx % VSL, u = 4 * (idx / VSL), v = v0 + vl;
      const bool ok = v < V;
      const float x4[4] = {ok ? xd[i].x : 0.f, ok ? xd[i].y : 0.f, ok ? xd[i].z : 0.f, ok ? xd[i].w : 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const __bf16 hi = (__bf16)x4[e];
        dth[(u + e) * PLD + vl] = hi;
        dtl[(u + e) * PLD + vl] = (__bf16)(x4[e] - (float)hi);
      }
    }
    __syncthreads();
#pragma unroll
    for (int vs = 0; vs < VSL / 16; ++vs) {
      const int vv = v0 + 16 * vs + 8 * hh;
      bf16x8 a = bf16x8{};
      if (tokq >= 0 && vv < V) a = *reinterpret_cast<const bf16x8*>(dorow + vv);  // V % 8 == 0
      const int c = 16 * vs + 8 * hh;
#pragma unroll
      for (int j = 0; j < NTW; ++j) {
        const int kt = pc + 2 * j;
        if (kt < KT) {
          const int o = (32 * kt + li) * PLD + c;
          aq[j] = mfma_bf16(a, *reinterpret_cast<const bf16x8*>(&sth[o]), aq[j]);
          aq[j] = mfma_bf16(a, *reinterpret_cast<const bf16x8*>(&stl[o]), aq[j]);
        }
      }
      const int o = (32 * pc + li) * PLD + c;
      ap = mfma_bf16(a, *reinterpret_cast<const bf16x8*>(&dth[o]), ap);
      ap = mfma_bf16(a, *reinterpret_cast<const bf16x8*>(&dtl[o]), ap);
    }
  }
  __syncthreads();
  // dQK = causal e^{G_t-G_u} dO D^T -> LDS [t][u], split.
  {
    const int u = 32 * pc + li;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = 32 * rt + acc_row(r, hh);
      const float x = u <= t ? __expf(gam_s[t] - gam_s[u]) * ap[r] : 0.f;
      const __bf16 hi = (__bf16)x;
      dth[t * PLD + u] = hi;
      dtl[t * PLD + u] = (__bf16)(x - (float)hi);
    }
  }
  __syncthreads();
  // dQn = e^G (dO S_n^T) + dQK Kn; Kn^T fragments (kcol) are the B operands.
  const __bf16* kcol = reinterpret_cast<const __bf16*>(sv.kcol) + ((int64_t)s * nch + n) * frag_col_elems(K, 8);
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    const int kt = pc + 2 * j;
    if (kt >= KT) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) aq[j][r] *= __expf(gam_s[32 * rt + acc_row(r, hh)]);
#pragma unroll
    for (int us = 0; us < R / 16; ++us) {
      const int o = (32 * rt + li) * PLD + 16 * us + 8 * hh;
      const bf16x8 kb = *reinterpret_cast<const bf16x8*>(kcol + ((kt * 4 + us) * 64 + l) * 8);
      aq[j] = mfma_bf16(*reinterpret_cast<const bf16x8*>(&dth[o]), kb, aq[j]);
      aq[j] = mfma_bf16(*reinterpret_cast<const bf16x8*>(&dtl[o]), kb, aq[j]);
    }
  }
  // Normalisation backward: q^ . dQn per row, then dq.
  float qe[NTW][16];
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    const int kt = pc + 2 * j, k = 32 * kt + li;
    float c[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {  // clamped loads first, masks after
      const int t = 32 * rt + acc_row(r, hh), tok = token_at(p, n, t);
      const bool ok = kt < KT && k < K && tok >= 0;
      qe[j][r] = op_load<bf16_t>(p.q, b, h, ok ? tok : 0, ok ? k : 0);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = 32 * rt + acc_row(r, hh), tok = token_at(p, n, t);
      const bool ok = kt < KT && k < K && tok >= 0;
      qe[j][r] = ok ? qe[j][r] * qrd_s[t] : 0.f;
      c[r] = qe[j][r] * aq[j][r];
    }
    const float sq = tile_row_sum(c, l);
    if ((l & 1) == 0 && kt < KT) atomicAdd(&qdot_s[32 * rt + acc_row(sum_index(l), hh)], sq);
  }
  __syncthreads();
  float* dq = reinterpret_cast<float*>(dqo.ptr) + op_base(dqo, b, h);
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    const int kt = pc + 2 * j, k = 32 * kt + li;
    if (kt >= KT || k >= K) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = 32 * rt + acc_row(r, hh), tok = token_at(p, n, t);
      if (tok >= 0)
        dq[(int64_t)tok * dqo.st + k] = (qnm_s[t] > 1e-6f ? aq[j][r] - qe[j][r] * qdot_s[t] : aq[j][r]) * qrd_s[t];
    }
  }
}

}  // namespace gpa

namespace {

using namespace gpa;

template <typename F>
int allow_lds_read(F kernel, size_t bytes) {
  if (bytes <= 65536) return GPA_HIP_OK;
  return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)bytes) == hipSuccess
             ? GPA_HIP_OK
             : fail(GPA_HIP_EHIP, "gdn_read: cannot raise the LDS limit");
}

int read_kmax(int k) { return k <= 64 ? 64 : (k <= 128 ? 128 : 256); }

int check_read(const gpa_gdn_problem* p, const gpa_gdn_saved* sv) {
  if (!p || !sv) return fail(GPA_HIP_EINVAL, "gdn_read: null problem or saved");
  if (p->batch < 1 || p->heads < 1 || p->tokens < 1 || p->chunk < 1 || p->chunk > GPA_CHUNK_ROWS ||
      p->offset < 0 || p->offset >= p->chunk)
    return fail(GPA_HIP_EINVAL, "gdn_read: bad shape");
  if (p->dtype != GPA_DTYPE_BF16 || p->kdim % 16 != 0 || p->kdim > 256 || p->vdim % 8 != 0 ||
      p->vdim > GPA_OUT_MFMA_MAX_V)
    return fail(GPA_HIP_EUNSUPPORTED, "gdn_read: needs bf16, key width a multiple of 16 up to 256 and value width "
                                      "a multiple of 8 up to 256");
  if (!p->q.ptr) return fail(GPA_HIP_EINVAL, "gdn_read: null query");
  if (!sv->kn || !sv->qn || !sv->delta || !sv->states || !sv->gam || !sv->kcol || !sv->qcol)
    return fail(GPA_HIP_EINVAL, "gdn_read: a saved buffer is null");
  return GPA_HIP_OK;
}

template <int KM>
int read_forward(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, gpa_operand out, int nch, hipStream_t st) {
  hipLaunchKernelGGL((gdn_prep_q<bf16_t, KM, true>), dim3(nch, p.batch * p.heads), dim3(ONT), 0, st, p, sv, nch);
  return launch_out_mfma<KM>(p, sv, out, nch, st);
}

template <int KM>
int read_backward(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, gpa_operand dout, gpa_operand dq, int nch,
                  hipStream_t st) {
  const size_t lds = ReadDqLayout<KM>::BYTES;
  if (int rc = allow_lds_read(gdn_read_dq_mfma<KM>, lds)) return rc;
  hipLaunchKernelGGL((gdn_read_dq_mfma<KM>), dim3(nch, p.batch * p.heads), dim3(ONT), lds, st, p, sv, dout, dq,
                     nch);
  return GPA_HIP_OK;
}

}  // namespace

extern "C" int gpa_gdn_read(const gpa_gdn_problem* problem, const gpa_gdn_saved* saved, gpa_operand out,
                            hipStream_t stream) {
  if (int rc = check_read(problem, saved)) return rc;
  if (!out.ptr) return fail(GPA_HIP_EINVAL, "gdn_read: null output");
  const int nch = gpa_gdn_nchunks(problem->tokens, problem->offset, problem->chunk);
  int rc;
  switch (read_kmax(problem->kdim)) {
    case 64: rc = read_forward<64>(*problem, *saved, out, nch, stream); break;
    case 128: rc = read_forward<128>(*problem, *saved, out, nch, stream); break;
    default: rc = read_forward<256>(*problem, *saved, out, nch, stream); break;
  }
  return rc ? rc : check_launch("gpa_gdn_read");
}

extern "C" int gpa_gdn_read_backward(const gpa_gdn_problem* problem, const gpa_gdn_saved* saved, gpa_operand dout,
                                     gpa_operand dq, hipStream_t stream) {
  if (int rc = check_read(problem, saved)) return rc;
  if (!dout.ptr || !dq.ptr) return fail(GPA_HIP_EINVAL, "gdn_read_backward: null dout or dq");
  const int nch = gpa_gdn_nchunks(problem->tokens, problem->offset, problem->chunk);
  int rc;
  switch (read_kmax(problem->kdim)) {
    case 64: rc = read_backward<64>(*problem, *saved, dout, dq, nch, stream); break;
    case 128: rc = read_backward<128>(*problem, *saved, dout, dq, nch, stream); break;
    default: rc = read_backward<256>(*problem, *saved, dout, dq, nch, stream); break;
  }
  return rc ? rc : check_launch("gpa_gdn_read_backward");
}
