// Sequential GDN state recurrences on bf16 MFMA (gfx950 v_mfma_f32_32x32x16_bf16).
//
// One block = one stream x 64 state columns, 4 waves.  The state tile lives in
// fp32 MFMA accumulators for the whole sequence; per chunk
//   forward:  D = U - W S                        (C x K) . (K x 64)
//             S = e^{G_C} S + Kn^T (diag(e^{G_C-G}) D)
//   backward: dD = dd0 + diag(e^{G_C-G}) (Kn dS)
//             dS = e^{G_C} dS + Qn^T (diag(e^G) dO) - W^T dD + dstates[n]
//
// Precision.  The recurrences cancel strongly when the keys of a stream are
// nearly parallel (relation memories at initialisation), so a plain bf16
// rounding of S or dS is not accurate enough for the carried state and its
// gradients.  Every fp32 operand x is therefore split into bf16 hi + lo
// (x - hi rounded again) and a product uses hi*hi + hi*lo + lo*hi, which keeps
// about 16 significant bits.  Normalised keys and queries are exact in bf16
// (the model rounds them to the activation dtype) and need no split.
//
// Latency.  The chain is sequential in the chunk index.  GEMM1 operands and
// per-row epilogue operands are loop-carried: the copy for the next chunk is
// issued right after its last use in the current one.  GEMM2 operands (and
// state-gradient injections) are issued at the top of their own iteration.
// Both loads are thus covered by about half a chunk of work.
//
// Layouts.  A operands come from the fp32 saved buffers (row-major [C][K]);
// B operands are staged transposed through LDS.  Accumulator layout of a
// 32x32 tile: element r of lane l is (row 8*(r/4) + 4*(l/32) + r%4, column l%32).
#include <hip/hip_runtime.h>

#include "gdn_common.h"

namespace gpa {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int MV = 64;        // state columns per block
constexpr int TPAD = 8;       // bf16 padding of transposed LDS rows (keeps 16-byte alignment)
constexpr int CT = R + TPAD;  // row stride of [64 cols][64 rows] transposed tiles

__device__ __forceinline__ int acc_row(int r, int l) { return 8 * (r >> 2) + 4 * (l >> 5) + (r & 3); }

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

struct Split8 {
  bf16x8 hi, lo;
};

__device__ __forceinline__ Split8 split8(const float (&x)[8], float scale) {
  Split8 s;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float v = x[e] * scale;
    s.hi[e] = (__bf16)v;
    s.lo[e] = (__bf16)(v - (float)s.hi[e]);
  }
  return s;
}

__device__ __forceinline__ bf16x8 exact8(const float (&x)[8]) {
  bf16x8 f;
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = (__bf16)x[e];
  return f;
}

// hi*hi + hi*lo + lo*hi
__device__ __forceinline__ f32x16 mfma3(const Split8& a, bf16x8 bh, bf16x8 bl, f32x16 c) {
  c = mfma(a.hi, bh, c);
  c = mfma(a.hi, bl, c);
  return mfma(a.lo, bh, c);
}

// Write a 32x32 fp32 tile, transposed and split into bf16 hi/lo, to
// hi[(col0 + col) * ld + row0 + row] and lo[...].
__device__ __forceinline__ void put_split_t(__bf16* hi, __bf16* lo, int ld, int row0, int col0, const f32x16& acc,
                                            int l) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    bf16x4 xh, xl;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float v = acc[4 * g + e];
      xh[e] = (__bf16)v;
      xl[e] = (__bf16)(v - (float)xh[e]);
    }
    const int off = (col0 + (l & 31)) * ld + row0 + 8 * g + 4 * (l >> 5);
    *reinterpret_cast<bf16x4*>(&hi[off]) = xh;
    *reinterpret_cast<bf16x4*>(&lo[off]) = xl;
  }
}

__device__ __forceinline__ bf16x8 lds_frag(const __bf16* lds, int ld, int col0, int k0, int l) {
  return *reinterpret_cast<const bf16x8*>(&lds[(col0 + (l & 31)) * ld + k0 + 8 * (l >> 5)]);
}

// 8 floats of a row-major fp32 [rows][K] matrix: row `row`, columns k0+8*(l/32)+0..7.
__device__ __forceinline__ void load_row8(float (&x)[8], const float* m, int K, int row, int k0, int l) {
  const float4* p = reinterpret_cast<const float4*>(m + (int64_t)row * K + k0 + 8 * (l >> 5));
  const float4 a = p[0], b = p[1];
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

// 8 floats of column k of a row-major fp32 [C][K] matrix: rows c0+8*(l/32)+0..7.
__device__ __forceinline__ void load_col8(float (&x)[8], const float* m, int K, int k, int c0, int l) {
  const int c = c0 + 8 * (l >> 5);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = m[(int64_t)(c + e) * K + k];
}

template <int KM>
__device__ __forceinline__ void fwd_load_w(float (&wr)[KM / 16][8], const gpa_gdn_saved& sv, int s, int n, int nch,
                                           int K, int rt, int l) {
  const float* wm = sv.w + rows_off(s, n, nch, 0, K);
#pragma unroll
  for (int ks = 0; ks < KM / 16; ++ks) {
    if (16 * ks < K) load_row8(wr[ks], wm, K, 32 * rt + (l & 31), 16 * ks, l);
  }
}

__device__ __forceinline__ void fwd_load_ug(float (&ur)[16], float (&gr)[16], float& gc, const gpa_gdn_saved& sv,
                                            int s, int n, int nch, int V, int rt, int v, int l) {
  const float* um = sv.u + rows_off(s, n, nch, 0, V);
  const float* gm = sv.gam + rows_off(s, n, nch, 0, 1);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int c = 32 * rt + acc_row(r, l);
    ur[r] = v < V ? um[(int64_t)c * V + v] : 0.f;
    gr[r] = gm[c];
  }
  gc = gm[R - 1];
}

}  // namespace

template <int KM>
__global__ __launch_bounds__(NT) void gdn_state_fwd_mfma(gpa_gdn_problem p, gpa_gdn_saved sv, int nch) {
  constexpr int KLD = KM + TPAD;
  constexpr int NRB = KM / 32 >= 4 ? KM / 128 : 1;  // 32-row blocks of the state per wave
  extern __shared__ __align__(16) unsigned char smem_raw[];
  __bf16* sh = reinterpret_cast<__bf16*>(smem_raw);  // [MV][KLD]  S^T hi
  __bf16* sl = sh + MV * KLD;                        // [MV][KLD]  S^T lo
  __bf16* dh = sl + MV * KLD;                        // [MV][CT]   (e^{G_C-G} D)^T hi
  __bf16* dl = dh + MV * CT;                         // [MV][CT]   lo
  const int s = blockIdx.y, b = s / p.heads, h = s % p.heads;
  const int K = p.kdim, V = p.vdim, tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int v0 = blockIdx.x * MV;
  const bool owns = (KM / 32 >= 4) || w < KM / 32;  // row blocks rb = w + 4*i
  const int rt = w >> 1, ct = w & 1;               // this wave's D tile
  const int vd = v0 + 32 * ct + (l & 31);          // D tile column
  f32x16 acc[NRB][2];
#pragma unroll
  for (int i = 0; i < NRB; ++i)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int k = 32 * (w + 4 * i) + acc_row(r, l), v = v0 + 32 * cb + (l & 31);
        acc[i][cb][r] = (owns && p.s0 && k < K && v < V)
            ? p.s0[(int64_t)b * p.s0_sb + (int64_t)h * p.s0_sh + (int64_t)k * V + v] : 0.f;
      }
  // Loop-carried operands: each is reloaded for chunk n+1 right after its
  // last use in chunk n, so its latency is covered by the rest of the chunk.
  float wr[KM / 16][8], ur[16], gr_[16], gcr;
  fwd_load_w<KM>(wr, sv, s, 0, nch, K, rt, l);
  fwd_load_ug(ur, gr_, gcr, sv, s, 0, nch, V, rt, vd, l);
  for (int n = 0; n < nch; ++n) {
    // This chunk's GEMM2 operands (Kn^T columns).
    float kf[NRB][R / 16][8];
    {
      const float* kn = sv.kn + rows_off(s, n, nch, 0, K);
#pragma unroll
      for (int i = 0; i < NRB; ++i) {
        const int k = 32 * (w + 4 * i) + (l & 31);
#pragma unroll
        for (int cs = 0; cs < R / 16; ++cs) {
          if (owns && k < K) load_col8(kf[i][cs], kn, K, k, 16 * cs, l);
          else
#pragma unroll
            for (int e = 0; e < 8; ++e) kf[i][cs][e] = 0.f;
        }
      }
    }
    // (a) S_n -> saved states and LDS (transposed, split).
    const int64_t so = state_off(s, n, nch, K, V);
    if (owns) {
#pragma unroll
      for (int i = 0; i < NRB; ++i)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          const int k0 = 32 * (w + 4 * i), v = v0 + 32 * cb + (l & 31);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int k = k0 + acc_row(r, l);
            if (k < K && v < V) sv.states[so + (int64_t)k * V + v] = acc[i][cb][r];
          }
          put_split_t(sh, sl, KLD, k0, 32 * cb, acc[i][cb], l);
        }
    }
    lds_barrier();
    // (c) D = U - W S for the (rt, ct) tile.
    f32x16 d = {};
#pragma unroll
    for (int ks = 0; ks < KM / 16; ++ks) {
      if (16 * ks < K) {
        const Split8 a = split8(wr[ks], 1.f);
        d = mfma3(a, lds_frag(sh, KLD, 32 * ct, 16 * ks, l), lds_frag(sl, KLD, 32 * ct, 16 * ks, l), d);
      }
    }
    if (n + 1 < nch) fwd_load_w<KM>(wr, sv, s, n + 1, nch, K, rt, l);
    {
      float* dm = sv.delta + rows_off(s, n, nch, 0, V);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int c = 32 * rt + acc_row(r, l);
        const float x = ur[r] - d[r];
        if (vd < V) dm[(int64_t)c * V + vd] = x;
        d[r] = x * __expf(gcr - gr_[r]);
      }
      put_split_t(dh, dl, CT, 32 * rt, 32 * ct, d, l);
    }
    const float decay = __expf(gcr);
    if (n + 1 < nch) fwd_load_ug(ur, gr_, gcr, sv, s, n + 1, nch, V, rt, vd, l);
    lds_barrier();
    // (e) S = e^{G_C} S + Kn^T (e^{G_C-G} D).
    if (owns) {
#pragma unroll
      for (int i = 0; i < NRB; ++i) {
        acc[i][0] *= decay;
        acc[i][1] *= decay;
#pragma unroll
        for (int cs = 0; cs < R / 16; ++cs) {
          const bf16x8 a = exact8(kf[i][cs]);
#pragma unroll
          for (int cb = 0; cb < 2; ++cb) {
            acc[i][cb] = mfma(a, lds_frag(dh, CT, 32 * cb, 16 * cs, l), acc[i][cb]);
            acc[i][cb] = mfma(a, lds_frag(dl, CT, 32 * cb, 16 * cs, l), acc[i][cb]);
          }
        }
      }
    }
    lds_barrier();
  }
  if (owns) {
#pragma unroll
    for (int i = 0; i < NRB; ++i)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const int v = v0 + 32 * cb + (l & 31);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int k = 32 * (w + 4 * i) + acc_row(r, l);
          if (k < K && v < V) sv.final[(int64_t)s * K * V + (int64_t)k * V + v] = acc[i][cb][r];
        }
      }
  }
}

namespace {

template <int KM>
__device__ __forceinline__ void bwd_load_k(float (&kr)[KM / 16][8], const gpa_gdn_saved& sv, int s, int n, int nch,
                                           int K, int rt, int l) {
  const float* kn = sv.kn + rows_off(s, n, nch, 0, K);
#pragma unroll
  for (int ks = 0; ks < KM / 16; ++ks) {
    if (16 * ks < K) load_row8(kr[ks], kn, K, 32 * rt + (l & 31), 16 * ks, l);
  }
}

__device__ __forceinline__ void bwd_load_rows(float (&d0r)[16], float (&dor)[16], float (&gr_)[16], float& gc,
                                              const gpa_gdn_problem& p, const gpa_gdn_saved& sv,
                                              const gpa_gdn_grads& gr, int s, int b, int h, int n, int nch, int V,
                                              int rt, int v, int l, bool has_q) {
  const float* d0 = gr.dd0 ? gr.dd0 + rows_off(s, n, nch, 0, V) : nullptr;
  const float* gm = sv.gam + rows_off(s, n, nch, 0, 1);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int c = 32 * rt + acc_row(r, l);
    d0r[r] = (d0 && v < V) ? d0[(int64_t)c * V + v] : 0.f;
    float o = 0.f;
    if (has_q && v < V) {
      const int t = token_at(p, n, c);
      if (t >= 0) o = op_load<bf16_t>(gr.dout, b, h, t, v);
    }
    dor[r] = o;
    gr_[r] = gm[c];
  }
  gc = gm[R - 1];
}

}  // namespace

template <int KM>
__global__ __launch_bounds__(NT) void gdn_state_bwd_mfma(gpa_gdn_problem p, gpa_gdn_saved sv, gpa_gdn_grads gr,
                                                          int nch) {
  constexpr int KLD = KM + TPAD;
  constexpr int NRB = KM / 32 >= 4 ? KM / 128 : 1;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  __bf16* sh = reinterpret_cast<__bf16*>(smem_raw);  // [MV][KLD]  dS^T hi
  __bf16* sl = sh + MV * KLD;                        // [MV][KLD]  lo
  __bf16* dh = sl + MV * KLD;                        // [MV][CT]   dD^T hi
  __bf16* dl = dh + MV * CT;                         // [MV][CT]   lo
  __bf16* oh = dl + MV * CT;                         // [MV][CT]   (e^G dO)^T hi
  __bf16* ol = oh + MV * CT;                         // [MV][CT]   lo
  const int s = blockIdx.y, b = s / p.heads, h = s % p.heads;
  const int K = p.kdim, V = p.vdim, tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int v0 = blockIdx.x * MV;
  const bool has_q = p.q.ptr != nullptr && gr.dout.ptr != nullptr;
  const bool owns = (KM / 32 >= 4) || w < KM / 32;
  const int rt = w >> 1, ct = w & 1;
  const int vd = v0 + 32 * ct + (l & 31);
  f32x16 acc[NRB][2];
#pragma unroll
  for (int i = 0; i < NRB; ++i)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int k = 32 * (w + 4 * i) + acc_row(r, l), v = v0 + 32 * cb + (l & 31);
        acc[i][cb][r] = (owns && gr.dfinal && k < K && v < V) ? gr.dfinal[(int64_t)s * K * V + (int64_t)k * V + v]
                                                              : 0.f;
      }
  // Loop-carried operands (see the forward kernel).
  float kr[KM / 16][8], d0r[16], dor[16], gr_[16], gcr;
  bwd_load_k<KM>(kr, sv, s, nch - 1, nch, K, rt, l);
  bwd_load_rows(d0r, dor, gr_, gcr, p, sv, gr, s, b, h, nch - 1, nch, V, rt, vd, l, has_q);
  for (int n = nch - 1; n >= 0; --n) {
    // This chunk's GEMM2 operands (W^T and Qn^T columns) and injections.
    const int64_t so = state_off(s, n, nch, K, V);
    float wf[NRB][R / 16][8], qf[NRB][R / 16][8], inj[NRB][2][16];
    {
      const float* wm = sv.w + rows_off(s, n, nch, 0, K);
      const float* qn = has_q ? sv.qn + rows_off(s, n, nch, 0, K) : nullptr;
#pragma unroll
      for (int i = 0; i < NRB; ++i) {
        const int k = 32 * (w + 4 * i) + (l & 31);
        const bool ok = owns && k < K;
#pragma unroll
        for (int cs = 0; cs < R / 16; ++cs) {
          if (ok) load_col8(wf[i][cs], wm, K, k, 16 * cs, l);
          else
#pragma unroll
            for (int e = 0; e < 8; ++e) wf[i][cs][e] = 0.f;
          if (ok && has_q) load_col8(qf[i][cs], qn, K, k, 16 * cs, l);
          else
#pragma unroll
            for (int e = 0; e < 8; ++e) qf[i][cs][e] = 0.f;
        }
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          const int v = v0 + 32 * cb + (l & 31);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int kk = 32 * (w + 4 * i) + acc_row(r, l);
            inj[i][cb][r] = (gr.dstates && owns && kk < K && v < V) ? gr.dstates[so + (int64_t)kk * V + v] : 0.f;
          }
        }
      }
    }
    // (a) dS -> dhend and LDS (transposed, split).
    if (owns) {
#pragma unroll
      for (int i = 0; i < NRB; ++i)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          const int k0 = 32 * (w + 4 * i), v = v0 + 32 * cb + (l & 31);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int k = k0 + acc_row(r, l);
            if (k < K && v < V) gr.dhend[so + (int64_t)k * V + v] = acc[i][cb][r];
          }
          put_split_t(sh, sl, KLD, k0, 32 * cb, acc[i][cb], l);
        }
    }
    lds_barrier();
    // (c) dD = dd0 + e^{G_C-G} (Kn dS); stage (e^G dO)^T.
    f32x16 d = {};
#pragma unroll
    for (int ks = 0; ks < KM / 16; ++ks) {
      if (16 * ks < K) {
        const bf16x8 a = exact8(kr[ks]);
        d = mfma(a, lds_frag(sh, KLD, 32 * ct, 16 * ks, l), d);
        d = mfma(a, lds_frag(sl, KLD, 32 * ct, 16 * ks, l), d);
      }
    }
    if (n > 0) bwd_load_k<KM>(kr, sv, s, n - 1, nch, K, rt, l);
    {
      float* ddm = gr.ddelta + rows_off(s, n, nch, 0, V);
      f32x16 o;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int c = 32 * rt + acc_row(r, l);
        const float x = d0r[r] + __expf(gcr - gr_[r]) * d[r];
        d[r] = x;
        if (vd < V) ddm[(int64_t)c * V + vd] = x;
        o[r] = __expf(gr_[r]) * dor[r];
      }
      put_split_t(dh, dl, CT, 32 * rt, 32 * ct, d, l);
      put_split_t(oh, ol, CT, 32 * rt, 32 * ct, o, l);
    }
    const float decay = __expf(gcr);
    if (n > 0) bwd_load_rows(d0r, dor, gr_, gcr, p, sv, gr, s, b, h, n - 1, nch, V, rt, vd, l, has_q);
    lds_barrier();
    // (e) dS = e^{G_C} dS + Qn^T (e^G dO) - W^T dD + dstates[n].
    if (owns) {
#pragma unroll
      for (int i = 0; i < NRB; ++i) {
        acc[i][0] *= decay;
        acc[i][1] *= decay;
#pragma unroll
        for (int cs = 0; cs < R / 16; ++cs) {
          const Split8 aw = split8(wf[i][cs], -1.f);
#pragma unroll
          for (int cb = 0; cb < 2; ++cb)
            acc[i][cb] = mfma3(aw, lds_frag(dh, CT, 32 * cb, 16 * cs, l), lds_frag(dl, CT, 32 * cb, 16 * cs, l),
                               acc[i][cb]);
          if (has_q) {
            const bf16x8 aq = exact8(qf[i][cs]);
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
              acc[i][cb] = mfma(aq, lds_frag(oh, CT, 32 * cb, 16 * cs, l), acc[i][cb]);
              acc[i][cb] = mfma(aq, lds_frag(ol, CT, 32 * cb, 16 * cs, l), acc[i][cb]);
            }
          }
        }
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][cb][r] += inj[i][cb][r];
      }
    }
    lds_barrier();
  }
  if (owns) {
#pragma unroll
    for (int i = 0; i < NRB; ++i)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const int v = v0 + 32 * cb + (l & 31);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int k = 32 * (w + 4 * i) + acc_row(r, l);
          if (k < K && v < V) gr.ds0[(int64_t)s * K * V + (int64_t)k * V + v] = acc[i][cb][r];
        }
      }
  }
}

namespace {

template <typename F>
int allow_lds_mfma(F kernel, size_t bytes) {
  if (bytes <= 65536) return GPA_HIP_OK;
  const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  return err == hipSuccess ? GPA_HIP_OK : fail(GPA_HIP_EHIP, "hipFuncSetAttribute(max dynamic LDS) failed");
}

}  // namespace

template <int KM>
int launch_state_fwd_mfma(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, int nch, hipStream_t st) {
  const size_t lds = sizeof(__bf16) * (2 * MV * (KM + TPAD) + 2 * MV * CT);
  if (int rc = allow_lds_mfma(gdn_state_fwd_mfma<KM>, lds)) return rc;
  hipLaunchKernelGGL((gdn_state_fwd_mfma<KM>), dim3((p.vdim + MV - 1) / MV, p.batch * p.heads), dim3(NT), lds, st,
                     p, sv, nch);
  return GPA_HIP_OK;
}

template <int KM>
int launch_state_bwd_mfma(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, const gpa_gdn_grads& gr, int nch,
                          hipStream_t st) {
  const size_t lds = sizeof(__bf16) * (2 * MV * (KM + TPAD) + 4 * MV * CT);
  if (int rc = allow_lds_mfma(gdn_state_bwd_mfma<KM>, lds)) return rc;
  hipLaunchKernelGGL((gdn_state_bwd_mfma<KM>), dim3((p.vdim + MV - 1) / MV, p.batch * p.heads), dim3(NT), lds, st,
                     p, sv, gr, nch);
  return GPA_HIP_OK;
}

template int launch_state_fwd_mfma<64>(const gpa_gdn_problem&, const gpa_gdn_saved&, int, hipStream_t);
template int launch_state_fwd_mfma<128>(const gpa_gdn_problem&, const gpa_gdn_saved&, int, hipStream_t);
template int launch_state_fwd_mfma<256>(const gpa_gdn_problem&, const gpa_gdn_saved&, int, hipStream_t);
template int launch_state_bwd_mfma<64>(const gpa_gdn_problem&, const gpa_gdn_saved&, const gpa_gdn_grads&, int,
                                       hipStream_t);
template int launch_state_bwd_mfma<128>(const gpa_gdn_problem&, const gpa_gdn_saved&, const gpa_gdn_grads&, int,
                                        hipStream_t);
template int launch_state_bwd_mfma<256>(const gpa_gdn_problem&, const gpa_gdn_saved&, const gpa_gdn_grads&, int,
                                        hipStream_t);

}  // namespace gpa
