// Sequential GDN state recurrences on bf16 MFMA (gfx950 v_mfma_f32_32x32x16_bf16).
//
// One block = one stream x 64 state columns, 4 waves.  The state tile lives in
// fp32 MFMA accumulators for the whole sequence; per chunk
//   forward:  D = U - W S                        (C x K) . (K x 64)
//             S = e^{G_C} S + Kn^T (diag(e^{G_C-G}) D)
//   backward: dD = dd0 + diag(e^{G_C-G}) (Kn dS)
//             dS = e^{G_C} dS + Qn^T o - W^T dD + dstates[n],   o = diag(e^G) dO
//
// Precision.  The recurrences cancel strongly when the keys of a stream are
// nearly parallel (relation memories at initialisation), so a plain bf16
// rounding of S or dS is not accurate enough for the carried state and its
// gradients.  Every fp32 operand x is split into bf16 hi + lo (x - hi rounded
// again) and a product uses hi*hi + hi*lo + lo*hi (about 16 significant
// bits).  Normalised keys and queries are exact in bf16 (the model rounds
// them to the activation dtype) and need no split.
//
// Memory.  Each chunk step is a dependent chain, and a wave can track only a
// bounded number of outstanding vector-memory instructions in order, so every
// global access is one 16-byte vector per lane: the matrix operands come as
// fragment-ordered bf16 written by the chunk kernel (gdn_prep), and all
// per-position data (U, D, dd0, o, dD) and the chunk-start states are stored
// value-major, which puts the four consecutive rows an accumulator lane owns
// in 16 contiguous bytes.  Operands that start the chunk (W or Kn rows, U,
// dd0, o, gates) are loop-carried and re-issued for the next chunk right
// after their last use; the GEMM2 operands of a chunk are issued at the top of
// its iteration.  B operands are staged transposed in LDS; barriers order LDS
// only (nothing global is read back in-kernel).
//
// Accumulator layout of a 32x32 tile: element r of lane l is
// (row 8*(r/4) + 4*(l/32) + r%4, column l%32).
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

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

struct Split8 {
  bf16x8 hi, lo;
};

__device__ __forceinline__ Split8 load_split(const __bf16* p) {
  Split8 s;
  s.hi = *reinterpret_cast<const bf16x8*>(p);
  s.lo = *reinterpret_cast<const bf16x8*>(p + 8);
  return s;
}

__device__ __forceinline__ Split8 negate(const Split8& a) {
  Split8 s;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    s.hi[e] = (__bf16)(-(float)a.hi[e]);
    s.lo[e] = (__bf16)(-(float)a.lo[e]);
  }
  return s;
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

// A value-major [V][R] tile column v, rows row0 + 8g + 4(l/32) + 0..3 for g < 4,
// as the 16 accumulator elements of lane l (zero when v >= V).
__device__ __forceinline__ void load_acc_vc(float (&x)[16], const float* m, int v, int V, int row0, int l) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
    if (v < V) q = *reinterpret_cast<const float4*>(m + (int64_t)v * R + row0 + 8 * g + 4 * (l >> 5));
    x[4 * g] = q.x; x[4 * g + 1] = q.y; x[4 * g + 2] = q.z; x[4 * g + 3] = q.w;
  }
}

__device__ __forceinline__ void store_acc_vc(float* m, int v, int V, int row0, const f32x16& x, int l) {
  if (v >= V) return;
#pragma unroll
  for (int g = 0; g < 4; ++g)
    *reinterpret_cast<float4*>(m + (int64_t)v * R + row0 + 8 * g + 4 * (l >> 5)) =
        make_float4(x[4 * g], x[4 * g + 1], x[4 * g + 2], x[4 * g + 3]);
}

// Value-major [V][K] state tile: rows k0 + 8g + 4(l/32) + 0..3, column v.
__device__ __forceinline__ void store_state(float* m, int v, int V, int K, int k0, const f32x16& x, int l) {
  if (v >= V) return;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int k = k0 + 8 * g + 4 * (l >> 5);
    if (k < K)
      *reinterpret_cast<float4*>(m + (int64_t)v * K + k) = make_float4(x[4 * g], x[4 * g + 1], x[4 * g + 2], x[4 * g + 3]);
  }
}

__device__ __forceinline__ void add_state(f32x16& x, const float* m, int v, int V, int K, int k0, int l) {
  if (v >= V) return;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int k = k0 + 8 * g + 4 * (l >> 5);
    if (k < K) {
      const float4 q = *reinterpret_cast<const float4*>(m + (int64_t)v * K + k);
      x[4 * g] += q.x; x[4 * g + 1] += q.y; x[4 * g + 2] += q.z; x[4 * g + 3] += q.w;
    }
  }
}

// Gates of the 16 accumulator rows of lane l (row block row0) and G_C.
__device__ __forceinline__ void load_gates(float (&g16)[16], float& gc, const float* gm, int row0, int l) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float4 q = *reinterpret_cast<const float4*>(gm + row0 + 8 * g + 4 * (l >> 5));
    g16[4 * g] = q.x; g16[4 * g + 1] = q.y; g16[4 * g + 2] = q.z; g16[4 * g + 3] = q.w;
  }
  gc = gm[R - 1];
}

// Key-major [K][V] state (initial state, final state and its gradient).
__device__ __forceinline__ void load_km(f32x16& x, const float* m, int64_t base, int v, int V, int K, int k0, int l) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int k = k0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    x[r] = (m && k < K && v < V) ? m[base + (int64_t)k * V + v] : 0.f;
  }
}

__device__ __forceinline__ void store_km(float* m, int64_t base, int v, int V, int K, int k0, const f32x16& x, int l) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int k = k0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    if (k < K && v < V) m[base + (int64_t)k * V + v] = x[r];
  }
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
  const int K16 = K / 16;
  const int v0 = blockIdx.x * MV;
  const bool owns = (KM / 32 >= 4) || w < KM / 32;  // row blocks rb = w + 4*i
  const int rt = w >> 1, ct = w & 1;               // this wave's D tile
  const int vd = v0 + 32 * ct + (l & 31);          // D tile column
  const int frag_row = frag_row_elems(K, 16), frag_col = frag_col_elems(K, 8);
  f32x16 acc[NRB][2];
#pragma unroll
  for (int i = 0; i < NRB; ++i)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
      load_km(acc[i][cb], p.s0, (int64_t)b * p.s0_sb + (int64_t)h * p.s0_sh, v0 + 32 * cb + (l & 31), V, K,
              owns ? 32 * (w + 4 * i) : K, l);

  // Loop-carried chunk-start operands.
  Split8 wr[KM / 16];
  float ur[16], gr_[16], gcr;
  auto load_start = [&](int n) {
    const __bf16* wf = reinterpret_cast<const __bf16*>(sv.wrow) + ((int64_t)s * nch + n) * frag_row;
#pragma unroll
    for (int ks = 0; ks < KM / 16; ++ks)
      if (ks < K16) wr[ks] = load_split(wf + ((rt * K16 + ks) * 64 + l) * 16);
    load_acc_vc(ur, sv.u + vc_off(s, n, nch, V), vd, V, 32 * rt, l);
    load_gates(gr_, gcr, sv.gam + rows_off(s, n, nch, 0, 1), 32 * rt, l);
  };
  load_start(0);
  for (int n = 0; n < nch; ++n) {
    const int64_t cid = (int64_t)s * nch + n;
    // This chunk's GEMM2 operands (Kn^T fragments).
    bf16x8 kf[NRB][R / 16];
    {
      const __bf16* kc = reinterpret_cast<const __bf16*>(sv.kcol) + cid * frag_col;
#pragma unroll
      for (int i = 0; i < NRB; ++i)
#pragma unroll
        for (int cs = 0; cs < R / 16; ++cs) {
          const int rb = w + 4 * i;
          if (owns && 32 * rb < K) kf[i][cs] = *reinterpret_cast<const bf16x8*>(kc + ((rb * 4 + cs) * 64 + l) * 8);
          else kf[i][cs] = bf16x8{};
        }
    }
    // (a) S_n -> saved states (value-major) and LDS (transposed, split).
    if (owns) {
      float* sm = sv.states + state_off(s, n, nch, K, V);
#pragma unroll
      for (int i = 0; i < NRB; ++i)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          const int k0 = 32 * (w + 4 * i);
          store_state(sm, v0 + 32 * cb + (l & 31), V, K, k0, acc[i][cb], l);
          put_split_t(sh, sl, KLD, k0, 32 * cb, acc[i][cb], l);
        }
    }
    lds_barrier();
    // (c) D = U - W S for the (rt, ct) tile.
    f32x16 d = {};
#pragma unroll
    for (int ks = 0; ks < KM / 16; ++ks)
      if (ks < K16) d = mfma3(wr[ks], lds_frag(sh, KLD, 32 * ct, 16 * ks, l), lds_frag(sl, KLD, 32 * ct, 16 * ks, l), d);
#pragma unroll
    for (int r = 0; r < 16; ++r) d[r] = ur[r] - d[r];
    store_acc_vc(sv.delta + vc_off(s, n, nch, V), vd, V, 32 * rt, d, l);
#pragma unroll
    for (int r = 0; r < 16; ++r) d[r] *= __expf(gcr - gr_[r]);
    put_split_t(dh, dl, CT, 32 * rt, 32 * ct, d, l);
    const float decay = __expf(gcr);
    if (n + 1 < nch) load_start(n + 1);
    lds_barrier();
    // (e) S = e^{G_C} S + Kn^T (e^{G_C-G} D).
    if (owns) {
#pragma unroll
      for (int i = 0; i < NRB; ++i) {
        acc[i][0] *= decay;
        acc[i][1] *= decay;
#pragma unroll
        for (int cs = 0; cs < R / 16; ++cs)
#pragma unroll
          for (int cb = 0; cb < 2; ++cb) {
            acc[i][cb] = mfma(kf[i][cs], lds_frag(dh, CT, 32 * cb, 16 * cs, l), acc[i][cb]);
            acc[i][cb] = mfma(kf[i][cs], lds_frag(dl, CT, 32 * cb, 16 * cs, l), acc[i][cb]);
          }
      }
    }
    lds_barrier();
  }
  if (owns) {
#pragma unroll
    for (int i = 0; i < NRB; ++i)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
        store_km(sv.final, (int64_t)s * K * V, v0 + 32 * cb + (l & 31), V, K, 32 * (w + 4 * i), acc[i][cb], l);
  }
}

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
  __bf16* oh = dl + MV * CT;                         // [MV][CT]   o^T hi
  __bf16* ol = oh + MV * CT;                         // [MV][CT]   lo
  const int s = blockIdx.y;
  const int K = p.kdim, V = p.vdim, tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int K16 = K / 16;
  const int v0 = blockIdx.x * MV;
  const bool has_q = p.q.ptr != nullptr && gr.dout.ptr != nullptr;
  const bool owns = (KM / 32 >= 4) || w < KM / 32;
  const int rt = w >> 1, ct = w & 1;
  const int vd = v0 + 32 * ct + (l & 31);
  const int frag_row = frag_row_elems(K, 8), frag_col = frag_col_elems(K, 8), frag_wcol = frag_col_elems(K, 16);
  f32x16 acc[NRB][2];
#pragma unroll
  for (int i = 0; i < NRB; ++i)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
      load_km(acc[i][cb], gr.dfinal, (int64_t)s * K * V, v0 + 32 * cb + (l & 31), V, K, owns ? 32 * (w + 4 * i) : K,
              l);

  // Loop-carried chunk-start operands.
  bf16x8 kr[KM / 16];
  float d0r[16], orr[16], gr_[16], gcr;
  auto load_start = [&](int n) {
    const __bf16* kf = reinterpret_cast<const __bf16*>(sv.krow) + ((int64_t)s * nch + n) * frag_row;
#pragma unroll
    for (int ks = 0; ks < KM / 16; ++ks)
      if (ks < K16) kr[ks] = *reinterpret_cast<const bf16x8*>(kf + ((rt * K16 + ks) * 64 + l) * 8);
    if (gr.dd0) {
      load_acc_vc(d0r, gr.dd0 + vc_off(s, n, nch, V), vd, V, 32 * rt, l);
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) d0r[r] = 0.f;
    }
    if (has_q) {
      load_acc_vc(orr, gr.o + vc_off(s, n, nch, V), vd, V, 32 * rt, l);
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) orr[r] = 0.f;
    }
    load_gates(gr_, gcr, sv.gam + rows_off(s, n, nch, 0, 1), 32 * rt, l);
  };
  load_start(nch - 1);
  for (int n = nch - 1; n >= 0; --n) {
    const int64_t cid = (int64_t)s * nch + n;
    // This chunk's GEMM2 operands (W^T, Qn^T fragments) and state injections.
    Split8 wf[NRB][R / 16];
    bf16x8 qf[NRB][R / 16];
    f32x16 inj[NRB][2];
    {
      const __bf16* wc = reinterpret_cast<const __bf16*>(sv.wcol) + cid * frag_wcol;
      const __bf16* qc = has_q ? reinterpret_cast<const __bf16*>(sv.qcol) + cid * frag_col : nullptr;
#pragma unroll
      for (int i = 0; i < NRB; ++i) {
        const int rb = w + 4 * i;
        const bool ok = owns && 32 * rb < K;
#pragma unroll
        for (int cs = 0; cs < R / 16; ++cs) {
          if (ok) wf[i][cs] = load_split(wc + ((rb * 4 + cs) * 64 + l) * 16);
          else wf[i][cs] = Split8{bf16x8{}, bf16x8{}};
          if (ok && has_q) qf[i][cs] = *reinterpret_cast<const bf16x8*>(qc + ((rb * 4 + cs) * 64 + l) * 8);
          else qf[i][cs] = bf16x8{};
        }
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          inj[i][cb] = f32x16{};
          if (gr.dstates && ok)
            add_state(inj[i][cb], gr.dstates + state_off(s, n, nch, K, V), v0 + 32 * cb + (l & 31), V, K, 32 * rb, l);
        }
      }
    }
    // (a) dS -> dhend (value-major) and LDS (transposed, split).
    if (owns) {
      float* dm = gr.dhend + state_off(s, n, nch, K, V);
#pragma unroll
      for (int i = 0; i < NRB; ++i)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          const int k0 = 32 * (w + 4 * i);
          store_state(dm, v0 + 32 * cb + (l & 31), V, K, k0, acc[i][cb], l);
          put_split_t(sh, sl, KLD, k0, 32 * cb, acc[i][cb], l);
        }
    }
    lds_barrier();
    // (c) dD = dd0 + e^{G_C-G} (Kn dS); stage o^T.
    f32x16 d = {};
#pragma unroll
    for (int ks = 0; ks < KM / 16; ++ks)
      if (ks < K16) {
        d = mfma(kr[ks], lds_frag(sh, KLD, 32 * ct, 16 * ks, l), d);
        d = mfma(kr[ks], lds_frag(sl, KLD, 32 * ct, 16 * ks, l), d);
      }
    f32x16 o;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      d[r] = d0r[r] + __expf(gcr - gr_[r]) * d[r];
      o[r] = orr[r];
    }
    store_acc_vc(gr.ddelta + vc_off(s, n, nch, V), vd, V, 32 * rt, d, l);
    put_split_t(dh, dl, CT, 32 * rt, 32 * ct, d, l);
    put_split_t(oh, ol, CT, 32 * rt, 32 * ct, o, l);
    const float decay = __expf(gcr);
    if (n > 0) load_start(n - 1);
    lds_barrier();
    // (e) dS = e^{G_C} dS + Qn^T o - W^T dD + dstates[n].
    if (owns) {
#pragma unroll
      for (int i = 0; i < NRB; ++i) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) acc[i][cb] = acc[i][cb] * decay + inj[i][cb];
#pragma unroll
        for (int cs = 0; cs < R / 16; ++cs) {
          const Split8 aw = negate(wf[i][cs]);
#pragma unroll
          for (int cb = 0; cb < 2; ++cb)
            acc[i][cb] = mfma3(aw, lds_frag(dh, CT, 32 * cb, 16 * cs, l), lds_frag(dl, CT, 32 * cb, 16 * cs, l),
                               acc[i][cb]);
          if (has_q) {
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
              acc[i][cb] = mfma(qf[i][cs], lds_frag(oh, CT, 32 * cb, 16 * cs, l), acc[i][cb]);
              acc[i][cb] = mfma(qf[i][cs], lds_frag(ol, CT, 32 * cb, 16 * cs, l), acc[i][cb]);
            }
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
      for (int cb = 0; cb < 2; ++cb)
        store_km(gr.ds0, (int64_t)s * K * V, v0 + 32 * cb + (l & 31), V, K, 32 * (w + 4 * i), acc[i][cb], l);
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
