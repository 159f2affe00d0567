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

// One lane's part of a planar split fragment (hi parts of the 64 lanes, then
// their lo parts): p points at the lane's hi part.
__device__ __forceinline__ Split8 load_split(const __bf16* p) {
  Split8 s;
  s.hi = *reinterpret_cast<const bf16x8*>(p);
  s.lo = *reinterpret_cast<const bf16x8*>(p + 512);
  return s;
}

// Write a 32x32 fp32 tile, transposed and split into bf16 hi/lo, to
// hi[(col0 + col) * ld + row0 + row] and lo[...].
__device__ __forceinline__ void put_split_t(__bf16* hi, __bf16* lo, int ld, int row0, int col0, const f32x16& acc,
                                            int l) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    uint2 xh, xl;
    bf2_split(acc[4 * g], acc[4 * g + 1], xh.x, xl.x);
    bf2_split(acc[4 * g + 2], acc[4 * g + 3], xh.y, xl.y);
    const int off = (col0 + (l & 31)) * ld + row0 + 8 * g + 4 * (l >> 5);
    *reinterpret_cast<uint2*>(&hi[off]) = xh;
    *reinterpret_cast<uint2*>(&lo[off]) = xl;
  }
}

__device__ __forceinline__ bf16x8 lds_frag(const __bf16* lds, int ld, int col0, int k0, int l) {
  return *reinterpret_cast<const bf16x8*>(&lds[(col0 + (l & 31)) * ld + k0 + 8 * (l >> 5)]);
}

// A value-major [V][R] tile column v, rows row0 + 8g + 4(l/32) + 0..3 for g < 4,
// as the 16 accumulator elements of lane l (zero when v >= V).  GUARD = false
// when the caller knows v < V.
template <bool GUARD = true>
__device__ __forceinline__ void load_acc_vc(float (&x)[16], const float* m, int v, int V, int row0, int l) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
    if (!GUARD || v < V) q = *reinterpret_cast<const float4*>(m + (int64_t)v * R + row0 + 8 * g + 4 * (l >> 5));
    x[4 * g] = q.x; x[4 * g + 1] = q.y; x[4 * g + 2] = q.z; x[4 * g + 3] = q.w;
  }
}

template <bool GUARD = true>
__device__ __forceinline__ void store_acc_vc(float* m, int v, int V, int row0, const f32x16& x, int l) {
  if (GUARD && v >= V) return;
#pragma unroll
  for (int g = 0; g < 4; ++g)
    *reinterpret_cast<float4*>(m + (int64_t)v * R + row0 + 8 * g + 4 * (l >> 5)) =
        make_float4(x[4 * g], x[4 * g + 1], x[4 * g + 2], x[4 * g + 3]);
}

// Value-major [V][K] state tile: rows k0 + 8g + 4(l/32) + 0..3, column v.
template <bool GUARD = true>
__device__ __forceinline__ void store_state(float* m, int v, int V, int K, int k0, const f32x16& x, int l) {
  if (GUARD && v >= V) return;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int k = k0 + 8 * g + 4 * (l >> 5);
    if (!GUARD || k < K)
      *reinterpret_cast<float4*>(m + (int64_t)v * K + k) = make_float4(x[4 * g], x[4 * g + 1], x[4 * g + 2], x[4 * g + 3]);
  }
}

template <bool GUARD = true>
__device__ __forceinline__ void add_state(f32x16& x, const float* m, int v, int V, int K, int k0, int l) {
  if (GUARD && v >= V) return;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int k = k0 + 8 * g + 4 * (l >> 5);
    if (!GUARD || k < K) {
      const float4 q = *reinterpret_cast<const float4*>(m + (int64_t)v * K + k);
      x[4 * g] += q.x; x[4 * g + 1] += q.y; x[4 * g + 2] += q.z; x[4 * g + 3] += q.w;
    }
  }
}

// The same elements, loaded (not added): nothing uses them here, so a
// prefetch stays in flight until its first use.
template <bool GUARD>
__device__ __forceinline__ void get_state(f32x16& x, const float* m, int v, int V, int K, int k0, int l) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int k = k0 + 8 * g + 4 * (l >> 5);
    if (!GUARD || (v < V && k < K)) {
      const float4 q = *reinterpret_cast<const float4*>(m + (int64_t)v * K + k);
      x[4 * g] = q.x; x[4 * g + 1] = q.y; x[4 * g + 2] = q.z; x[4 * g + 3] = q.w;
    } else {
      x[4 * g] = x[4 * g + 1] = x[4 * g + 2] = x[4 * g + 3] = 0.f;
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
// The 16 loads are unconditional (out-of-range elements read element (0, 0))
// and masked afterwards, so that they are in flight together.
__device__ __forceinline__ void load_km(f32x16& x, const float* m, int64_t base, int v, int V, int K, int k0, int l) {
  if (!m) {
    x = f32x16{};
    return;
  }
  float t[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int k = k0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    const bool ok = k < K && v < V;
    t[r] = m[base + (ok ? (int64_t)k * V + v : 0)];
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int k = k0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    x[r] = (k < K && v < V) ? t[r] : 0.f;
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

// Chunk operand addresses.  `Fast` kernels assume K == KM and V % 64 == 0, so
// every fragment and column they touch exists and the chunk loop is straight
// line code; the general instantiation guards k steps, row blocks and
// columns.
template <int KM, bool FAST>
struct Shape {
  int K, V, K16;
  __device__ __forceinline__ Shape(const gpa_gdn_problem& p)
      : K(FAST ? KM : p.kdim), V(p.vdim), K16((FAST ? KM : p.kdim) / 16) {}
  __device__ __forceinline__ bool kstep(int ks) const { return FAST || ks < K16; }
  __device__ __forceinline__ bool rows(int rb) const { return FAST || 32 * rb < K; }
  __device__ __forceinline__ bool col(int v) const { return FAST || v < V; }
};

// Loads whose next-chunk copy is issued right after the last use of the
// current one: with every operand reloaded as soon as it is dead, each load
// has a whole chunk step to arrive, and no extra registers are needed.
template <int KM, bool FAST>
__device__ __forceinline__ void state_fwd_mfma_run(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, int nch, int bx,
                                                   int s) {
  constexpr int KLD = KM + TPAD;
  constexpr int NRB = KM / 32 >= 4 ? KM / 128 : 1;  // 32-row blocks of the state per wave
  extern __shared__ __align__(16) unsigned char smem_raw[];
  __bf16* sh = reinterpret_cast<__bf16*>(smem_raw);  // [MV][KLD]  S^T hi
  __bf16* sl = sh + MV * KLD;                        // [MV][KLD]  S^T lo
  __bf16* dh = sl + MV * KLD;                        // [MV][CT]   (e^{G_C-G} D)^T hi
  __bf16* dl = dh + MV * CT;                         // [MV][CT]   lo
  const Shape<KM, FAST> sp(p);
  const int b = s / p.heads, h = s % p.heads;
  const int K = sp.K, V = sp.V, tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int v0 = bx * MV;
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

  const __bf16* wrow = reinterpret_cast<const __bf16*>(sv.wrow) + (int64_t)s * nch * frag_row;
  const __bf16* kcol = reinterpret_cast<const __bf16*>(sv.kcol) + (int64_t)s * nch * frag_col;
  auto w_at = [&](int n, int ks) { return wrow + (int64_t)n * frag_row + (rt * sp.K16 + ks) * 1024 + l * 8; };
  auto k_at = [&](int n, int rb, int cs) { return kcol + (int64_t)n * frag_col + ((rb * 4 + cs) * 64 + l) * 8; };
  Split8 wr[KM / 16];
  bf16x8 kf[NRB][R / 16];
  float ur[16], gr_[16], gcr;
#pragma unroll
  for (int ks = 0; ks < KM / 16; ++ks)
    if (sp.kstep(ks)) wr[ks] = load_split(w_at(0, ks));
#pragma unroll
  for (int i = 0; i < NRB; ++i)
#pragma unroll
    for (int cs = 0; cs < R / 16; ++cs)
      kf[i][cs] = owns && sp.rows(w + 4 * i) ? *reinterpret_cast<const bf16x8*>(k_at(0, w + 4 * i, cs)) : bf16x8{};
  load_ufrag<!FAST>(ur, sv.u + ufrag_off(s, 0, nch, V), (v0 + 32 * ct) >> 5, ufrag_v(V) >> 5, rt, l);
  load_gates(gr_, gcr, sv.gam + rows_off(s, 0, nch, 0, 1), 32 * rt, l);

  for (int n = 0; n < nch; ++n) {
    const int nn = n + 1 < nch ? n + 1 : n;  // operands of the next chunk (reloaded once at the end)
    // (a) S_n -> saved states (value-major) and LDS (transposed, split).
    if (owns) {
      float* sm = sv.states + state_off(s, n, nch, K, V);
#pragma unroll
      for (int i = 0; i < NRB; ++i)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          const int k0 = 32 * (w + 4 * i);
          if (sp.rows(w + 4 * i)) {
            store_state<!FAST>(sm, v0 + 32 * cb + (l & 31), V, K, k0, acc[i][cb], l);
            put_split_t(sh, sl, KLD, k0, 32 * cb, acc[i][cb], l);
          }
        }
    }
    lds_barrier();
    // (c) D = U - W S for the (rt, ct) tile; each W fragment is reloaded once used.
    // Two accumulation chains (hi*hi + lo*hi, hi*lo), and the LDS fragments of
    // the next k step are read while the current one multiplies.
    f32x16 d;
    {
      f32x16 d1 = {}, d2 = {};
      bf16x8 fb[2][2];
      fb[0][0] = lds_frag(sh, KLD, 32 * ct, 0, l);
      fb[0][1] = lds_frag(sl, KLD, 32 * ct, 0, l);
#pragma unroll
      for (int ks = 0; ks < KM / 16; ++ks)
        if (sp.kstep(ks)) {
          if (ks + 1 < KM / 16 && sp.kstep(ks + 1)) {
            fb[(ks + 1) & 1][0] = lds_frag(sh, KLD, 32 * ct, 16 * (ks + 1), l);
            fb[(ks + 1) & 1][1] = lds_frag(sl, KLD, 32 * ct, 16 * (ks + 1), l);
          }
          const bf16x8 bh = fb[ks & 1][0], bl = fb[ks & 1][1];
          d1 = mfma(wr[ks].hi, bh, d1);
          d2 = mfma(wr[ks].hi, bl, d2);
          d1 = mfma(wr[ks].lo, bh, d1);
          wr[ks] = load_split(w_at(nn, ks));
        }
      d = d1 + d2;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) d[r] = ur[r] - d[r];
    load_ufrag<!FAST>(ur, sv.u + ufrag_off(s, nn, nch, V), (v0 + 32 * ct) >> 5, ufrag_v(V) >> 5, rt, l);
    store_acc_vc<!FAST>(sv.delta + vc_off(s, n, nch, V), vd, V, 32 * rt, d, l);
#pragma unroll
    for (int r = 0; r < 16; ++r) d[r] *= __expf(gcr - gr_[r]);
    const float decay = __expf(gcr);
    load_gates(gr_, gcr, sv.gam + rows_off(s, nn, nch, 0, 1), 32 * rt, l);
    put_split_t(dh, dl, CT, 32 * rt, 32 * ct, d, l);
    lds_barrier();
    // (e) S = e^{G_C} S + Kn^T (e^{G_C-G} D); each Kn^T fragment is reloaded once used.
    // The next (a) writes only sh/sl, which no wave reads after the barrier above,
    // and the next (c) epilogue writes dh/dl only after the next barrier, so the
    // step needs no closing barrier.
    if (owns) {
#pragma unroll
      for (int i = 0; i < NRB; ++i) {
        acc[i][0] *= decay;
        acc[i][1] *= decay;
      }
      bf16x8 fb[2][2][2];  // [buffer][cb][hi, lo]
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        fb[0][cb][0] = lds_frag(dh, CT, 32 * cb, 0, l);
        fb[0][cb][1] = lds_frag(dl, CT, 32 * cb, 0, l);
      }
#pragma unroll
      for (int cs = 0; cs < R / 16; ++cs) {
        if (cs + 1 < R / 16) {
#pragma unroll
          for (int cb = 0; cb < 2; ++cb) {
            fb[(cs + 1) & 1][cb][0] = lds_frag(dh, CT, 32 * cb, 16 * (cs + 1), l);
            fb[(cs + 1) & 1][cb][1] = lds_frag(dl, CT, 32 * cb, 16 * (cs + 1), l);
          }
        }
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
          for (int i = 0; i < NRB; ++i)
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) acc[i][cb] = mfma(kf[i][cs], fb[cs & 1][cb][h2], acc[i][cb]);
#pragma unroll
        for (int i = 0; i < NRB; ++i)
          if (sp.rows(w + 4 * i)) kf[i][cs] = *reinterpret_cast<const bf16x8*>(k_at(nn, w + 4 * i, cs));
      }
    }
  }
  if (owns) {
#pragma unroll
    for (int i = 0; i < NRB; ++i)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
        store_km(sv.final, (int64_t)s * K * V, v0 + 32 * cb + (l & 31), V, K, 32 * (w + 4 * i), acc[i][cb], l);
  }
}

template <int KM, bool FAST, bool HAS_Q, bool HAS_INJ>
__device__ __forceinline__ void state_bwd_mfma_run(const gpa_gdn_problem& p, const gpa_gdn_saved& sv,
                                                   const gpa_gdn_grads& gr, int nch, int bx, int s) {
  constexpr int KLD = KM + TPAD;
  constexpr int NRB = KM / 32 >= 4 ? KM / 128 : 1;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  __bf16* sh = reinterpret_cast<__bf16*>(smem_raw);  // [MV][KLD]  dS^T hi
  __bf16* sl = sh + MV * KLD;                        // [MV][KLD]  lo
  __bf16* dh = sl + MV * KLD;                        // [MV][CT]   -dD^T hi
  __bf16* dl = dh + MV * CT;                         // [MV][CT]   lo
  __bf16* oh = dl + MV * CT;                         // [MV][CT]   o^T hi
  __bf16* ol = oh + MV * CT;                         // [MV][CT]   lo
  const Shape<KM, FAST> sp(p);
  const int K = sp.K, V = sp.V, tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int v0 = bx * MV;
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

  const __bf16* krow = reinterpret_cast<const __bf16*>(sv.krow) + (int64_t)s * nch * frag_row;
  const __bf16* wcol = reinterpret_cast<const __bf16*>(sv.wcol) + (int64_t)s * nch * frag_wcol;
  const __bf16* qcol = HAS_Q ? reinterpret_cast<const __bf16*>(sv.qcol) + (int64_t)s * nch * frag_col : nullptr;
  auto k_at = [&](int n, int ks) { return krow + (int64_t)n * frag_row + ((rt * sp.K16 + ks) * 64 + l) * 8; };
  auto w_at = [&](int n, int rb, int cs) { return wcol + (int64_t)n * frag_wcol + (rb * 4 + cs) * 1024 + l * 8; };
  auto q_at = [&](int n, int rb, int cs) { return qcol + (int64_t)n * frag_col + ((rb * 4 + cs) * 64 + l) * 8; };
  bf16x8 kr[KM / 16];
  Split8 wf[NRB][R / 16];
  bf16x8 qf[HAS_Q ? NRB : 1][R / 16];
  f32x16 inj[HAS_INJ ? NRB : 1][2];
  float d0r[16], orr[16], gr_[16], gcr;
  auto load_inj = [&](int n) {
    if constexpr (HAS_INJ) {
#pragma unroll
      for (int i = 0; i < NRB; ++i)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          if (owns && sp.rows(w + 4 * i))
            get_state<!FAST>(inj[i][cb], gr.dstates + state_off(s, n, nch, K, V), v0 + 32 * cb + (l & 31), V, K,
                             32 * (w + 4 * i), l);
          else
            inj[i][cb] = f32x16{};
        }
    }
  };
  {
    const int n = nch - 1;
#pragma unroll
    for (int ks = 0; ks < KM / 16; ++ks)
      if (sp.kstep(ks)) kr[ks] = *reinterpret_cast<const bf16x8*>(k_at(n, ks));
#pragma unroll
    for (int i = 0; i < NRB; ++i) {
      const bool ok = owns && sp.rows(w + 4 * i);
#pragma unroll
      for (int cs = 0; cs < R / 16; ++cs) {
        wf[i][cs] = ok ? load_split(w_at(n, w + 4 * i, cs)) : Split8{bf16x8{}, bf16x8{}};
        if constexpr (HAS_Q) qf[i][cs] = ok ? *reinterpret_cast<const bf16x8*>(q_at(n, w + 4 * i, cs)) : bf16x8{};
      }
    }
    if constexpr (HAS_Q) {
      load_ufrag<!FAST>(d0r, gr.dd0 + ufrag_off(s, n, nch, V), (v0 + 32 * ct) >> 5, ufrag_v(V) >> 5, rt, l);
      load_ufrag<!FAST>(orr, gr.o + ufrag_off(s, n, nch, V), (v0 + 32 * ct) >> 5, ufrag_v(V) >> 5, rt, l);
    }
    load_gates(gr_, gcr, sv.gam + rows_off(s, n, nch, 0, 1), 32 * rt, l);
    load_inj(n);
  }
  for (int n = nch - 1; n >= 0; --n) {
    const int nn = n > 0 ? n - 1 : 0;  // operands of the next (earlier) chunk
    // (a) dS -> dhend (value-major) and LDS (transposed, split).
    if (owns) {
      float* dm = gr.dhend + state_off(s, n, nch, K, V);
#pragma unroll
      for (int i = 0; i < NRB; ++i)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          const int k0 = 32 * (w + 4 * i);
          if (sp.rows(w + 4 * i)) {
            store_state<!FAST>(dm, v0 + 32 * cb + (l & 31), V, K, k0, acc[i][cb], l);
            put_split_t(sh, sl, KLD, k0, 32 * cb, acc[i][cb], l);
          }
        }
    }
    lds_barrier();
    // (c) dD = dd0 + e^{G_C-G} (Kn dS); stage o^T.  Kn fragments are reloaded once
    // used; hi and lo parts accumulate in separate chains and the next k step's
    // LDS fragments are read while the current one multiplies.
    f32x16 d;
    {
      f32x16 d1 = {}, d2 = {};
      bf16x8 fb[2][2];
      fb[0][0] = lds_frag(sh, KLD, 32 * ct, 0, l);
      fb[0][1] = lds_frag(sl, KLD, 32 * ct, 0, l);
#pragma unroll
      for (int ks = 0; ks < KM / 16; ++ks)
        if (sp.kstep(ks)) {
          if (ks + 1 < KM / 16 && sp.kstep(ks + 1)) {
            fb[(ks + 1) & 1][0] = lds_frag(sh, KLD, 32 * ct, 16 * (ks + 1), l);
            fb[(ks + 1) & 1][1] = lds_frag(sl, KLD, 32 * ct, 16 * (ks + 1), l);
          }
          d1 = mfma(kr[ks], fb[ks & 1][0], d1);
          d2 = mfma(kr[ks], fb[ks & 1][1], d2);
          kr[ks] = *reinterpret_cast<const bf16x8*>(k_at(nn, ks));
        }
      d = d1 + d2;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) d[r] = (HAS_Q ? d0r[r] : 0.f) + __expf(gcr - gr_[r]) * d[r];
    const float decay = __expf(gcr);
    load_gates(gr_, gcr, sv.gam + rows_off(s, nn, nch, 0, 1), 32 * rt, l);
    store_acc_vc<!FAST>(gr.ddelta + vc_off(s, n, nch, V), vd, V, 32 * rt, d, l);
    put_split_t(dh, dl, CT, 32 * rt, 32 * ct, -d, l);  // -dD: (e) adds W^T (-dD)
    if constexpr (HAS_Q) {
      f32x16 o;
#pragma unroll
      for (int r = 0; r < 16; ++r) o[r] = orr[r];
      put_split_t(oh, ol, CT, 32 * rt, 32 * ct, o, l);
      load_ufrag<!FAST>(d0r, gr.dd0 + ufrag_off(s, nn, nch, V), (v0 + 32 * ct) >> 5, ufrag_v(V) >> 5, rt, l);
      load_ufrag<!FAST>(orr, gr.o + ufrag_off(s, nn, nch, V), (v0 + 32 * ct) >> 5, ufrag_v(V) >> 5, rt, l);
    }
    lds_barrier();
    // (e) dS = e^{G_C} dS + Qn^T o - W^T dD + dstates[n]; fragments are reloaded once
    // used.  As in the forward kernel, no closing barrier is needed: the next (a)
    // writes sh/sl only, and the next (c) epilogue writes dh..ol after a barrier.
    if (owns) {
#pragma unroll
      for (int i = 0; i < NRB; ++i)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          acc[i][cb] *= decay;
          if constexpr (HAS_INJ) acc[i][cb] += inj[i][cb];
        }
      constexpr int NF = HAS_Q ? 4 : 2;  // -dD hi, lo, o hi, lo
      bf16x8 fb[2][2][NF];                // [buffer][cb][part]
      auto read_b = [&](bf16x8 (&f)[2][NF], int cs) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          f[cb][0] = lds_frag(dh, CT, 32 * cb, 16 * cs, l);
          f[cb][1] = lds_frag(dl, CT, 32 * cb, 16 * cs, l);
          if constexpr (HAS_Q) {
            f[cb][2] = lds_frag(oh, CT, 32 * cb, 16 * cs, l);
            f[cb][3] = lds_frag(ol, CT, 32 * cb, 16 * cs, l);
          }
        }
      };
      read_b(fb[0], 0);
#pragma unroll
      for (int cs = 0; cs < R / 16; ++cs) {
        if (cs + 1 < R / 16) read_b(fb[(cs + 1) & 1], cs + 1);
        const auto& f = fb[cs & 1];
        // W^T (-dD): hi*hi, hi*lo, lo*hi; then Qn^T o: q*hi, q*lo.  The chains of
        // the (row block, column block) tiles are interleaved.
#pragma unroll
        for (int i = 0; i < NRB; ++i)
#pragma unroll
          for (int cb = 0; cb < 2; ++cb) acc[i][cb] = mfma(wf[i][cs].hi, f[cb][0], acc[i][cb]);
#pragma unroll
        for (int i = 0; i < NRB; ++i)
#pragma unroll
          for (int cb = 0; cb < 2; ++cb) acc[i][cb] = mfma(wf[i][cs].hi, f[cb][1], acc[i][cb]);
#pragma unroll
        for (int i = 0; i < NRB; ++i)
#pragma unroll
          for (int cb = 0; cb < 2; ++cb) acc[i][cb] = mfma(wf[i][cs].lo, f[cb][0], acc[i][cb]);
#pragma unroll
        for (int i = 0; i < NRB; ++i)
          if (sp.rows(w + 4 * i)) wf[i][cs] = load_split(w_at(nn, w + 4 * i, cs));
        if constexpr (HAS_Q) {
#pragma unroll
          for (int h2 = 2; h2 < 4; ++h2)
#pragma unroll
            for (int i = 0; i < NRB; ++i)
#pragma unroll
              for (int cb = 0; cb < 2; ++cb) acc[i][cb] = mfma(qf[i][cs], f[cb][h2], acc[i][cb]);
#pragma unroll
          for (int i = 0; i < NRB; ++i)
            if (sp.rows(w + 4 * i)) qf[i][cs] = *reinterpret_cast<const bf16x8*>(q_at(nn, w + 4 * i, cs));
        }
      }
    }
    load_inj(nn);
  }
  if (owns) {
#pragma unroll
    for (int i = 0; i < NRB; ++i)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
        store_km(gr.ds0, (int64_t)s * K * V, v0 + 32 * cb + (l & 31), V, K, 32 * (w + 4 * i), acc[i][cb], l);
  }
}

template <int KM, bool FAST>
__global__ __launch_bounds__(NT) void gdn_state_fwd_mfma(gpa_gdn_problem p, gpa_gdn_saved sv, int nch) {
  state_fwd_mfma_run<KM, FAST>(p, sv, nch, blockIdx.x, blockIdx.y);
}

template <int KM, bool FAST, bool HAS_Q, bool HAS_INJ>
__global__ __launch_bounds__(NT) void gdn_state_bwd_mfma(gpa_gdn_problem p, gpa_gdn_saved sv, gpa_gdn_grads gr,
                                                          int nch) {
  state_bwd_mfma_run<KM, FAST, HAS_Q, HAS_INJ>(p, sv, gr, nch, blockIdx.x, blockIdx.y);
}

typedef const __attribute__((address_space(4))) MfmaPack* MfmaPackPtr;

// The pack entry of this workgroup (the pack is the kernel's only argument).
__device__ __forceinline__ int mfma_pack_entry(MfmaPackPtr kp) {
  int pi = 0;
#pragma unroll 1
  for (int i = 1; i < kp->n; ++i)
    if ((int)blockIdx.x >= kp->wg0[i]) pi = i;
  return pi;
}

template <int KM, bool FAST>
__global__ __launch_bounds__(NT) void gdn_state_fwd_mfma_pack(MfmaPack pk) {
  const MfmaPackPtr kp = (MfmaPackPtr)__builtin_amdgcn_kernarg_segment_ptr();
  const int pi = mfma_pack_entry(kp);
  gpa_gdn_problem p;
  gpa_gdn_saved sv;
  kernarg_copy(p, &kp->p[pi]);
  kernarg_copy(sv, &kp->sv[pi]);
  const int local = (int)blockIdx.x - kp->wg0[pi], nvb = kp->nvb[pi];
  state_fwd_mfma_run<KM, FAST>(p, sv, kp->nch[pi], local % nvb, local / nvb);
}

template <int KM, bool FAST, bool HAS_Q, bool HAS_INJ>
__global__ __launch_bounds__(NT) void gdn_state_bwd_mfma_pack(MfmaPack pk) {
  const MfmaPackPtr kp = (MfmaPackPtr)__builtin_amdgcn_kernarg_segment_ptr();
  const int pi = mfma_pack_entry(kp);
  gpa_gdn_problem p;
  gpa_gdn_saved sv;
  gpa_gdn_grads gr;
  kernarg_copy(p, &kp->p[pi]);
  kernarg_copy(sv, &kp->sv[pi]);
  kernarg_copy(gr, &kp->gr[pi]);
  const int local = (int)blockIdx.x - kp->wg0[pi], nvb = kp->nvb[pi];
  state_bwd_mfma_run<KM, FAST, HAS_Q, HAS_INJ>(p, sv, gr, kp->nch[pi], local % nvb, local / nvb);
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
  const dim3 grid((p.vdim + MV - 1) / MV, p.batch * p.heads);
  if (p.kdim == KM && p.vdim % MV == 0) {
    if (int rc = allow_lds_mfma(gdn_state_fwd_mfma<KM, true>, lds)) return rc;
    hipLaunchKernelGGL((gdn_state_fwd_mfma<KM, true>), grid, dim3(NT), lds, st, p, sv, nch);
  } else {
    if (int rc = allow_lds_mfma(gdn_state_fwd_mfma<KM, false>, lds)) return rc;
    hipLaunchKernelGGL((gdn_state_fwd_mfma<KM, false>), grid, dim3(NT), lds, st, p, sv, nch);
  }
  return GPA_HIP_OK;
}

template <int KM, bool FAST, bool HAS_Q, bool HAS_INJ>
int launch_bwd(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, const gpa_gdn_grads& gr, int nch, hipStream_t st) {
  const size_t lds = sizeof(__bf16) * (2 * MV * (KM + TPAD) + 4 * MV * CT);
  if (int rc = allow_lds_mfma(gdn_state_bwd_mfma<KM, FAST, HAS_Q, HAS_INJ>, lds)) return rc;
  hipLaunchKernelGGL((gdn_state_bwd_mfma<KM, FAST, HAS_Q, HAS_INJ>), dim3((p.vdim + MV - 1) / MV, p.batch * p.heads),
                     dim3(NT), lds, st, p, sv, gr, nch);
  return GPA_HIP_OK;
}

template <int KM, bool FAST>
int launch_bwd_flags(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, const gpa_gdn_grads& gr, int nch,
                     hipStream_t st) {
  const bool has_q = p.q.ptr != nullptr && gr.dout.ptr != nullptr, has_inj = gr.dstates != nullptr;
  if (has_q)
    return has_inj ? launch_bwd<KM, FAST, true, true>(p, sv, gr, nch, st)
                   : launch_bwd<KM, FAST, true, false>(p, sv, gr, nch, st);
  return has_inj ? launch_bwd<KM, FAST, false, true>(p, sv, gr, nch, st)
                 : launch_bwd<KM, FAST, false, false>(p, sv, gr, nch, st);
}

template <int KM>
int launch_state_bwd_mfma(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, const gpa_gdn_grads& gr, int nch,
                          hipStream_t st) {
  return p.kdim == KM && p.vdim % MV == 0 ? launch_bwd_flags<KM, true>(p, sv, gr, nch, st)
                                          : launch_bwd_flags<KM, false>(p, sv, gr, nch, st);
}

int mfma_state_workgroups(const gpa_gdn_problem& p) { return ((p.vdim + MV - 1) / MV) * p.batch * p.heads; }

template <int KM>
int launch_state_fwd_mfma_pack(const MfmaPack& pk, int total, bool fast, hipStream_t st) {
  const size_t lds = sizeof(__bf16) * (2 * MV * (KM + TPAD) + 2 * MV * CT);
  if (fast) {
    if (int rc = allow_lds_mfma(gdn_state_fwd_mfma_pack<KM, true>, lds)) return rc;
    hipLaunchKernelGGL((gdn_state_fwd_mfma_pack<KM, true>), dim3(total), dim3(NT), lds, st, pk);
  } else {
    if (int rc = allow_lds_mfma(gdn_state_fwd_mfma_pack<KM, false>, lds)) return rc;
    hipLaunchKernelGGL((gdn_state_fwd_mfma_pack<KM, false>), dim3(total), dim3(NT), lds, st, pk);
  }
  return GPA_HIP_OK;
}

namespace {
template <int KM, bool FAST, bool HAS_Q, bool HAS_INJ>
int launch_bwd_pack(const MfmaPack& pk, int total, hipStream_t st) {
  const size_t lds = sizeof(__bf16) * (2 * MV * (KM + TPAD) + 4 * MV * CT);
  if (int rc = allow_lds_mfma(gdn_state_bwd_mfma_pack<KM, FAST, HAS_Q, HAS_INJ>, lds)) return rc;
  hipLaunchKernelGGL((gdn_state_bwd_mfma_pack<KM, FAST, HAS_Q, HAS_INJ>), dim3(total), dim3(NT), lds, st, pk);
  return GPA_HIP_OK;
}
template <int KM, bool FAST>
int launch_bwd_pack_flags(const MfmaPack& pk, int total, bool has_q, bool has_inj, hipStream_t st) {
  if (has_q)
    return has_inj ? launch_bwd_pack<KM, FAST, true, true>(pk, total, st)
                   : launch_bwd_pack<KM, FAST, true, false>(pk, total, st);
  return has_inj ? launch_bwd_pack<KM, FAST, false, true>(pk, total, st)
                 : launch_bwd_pack<KM, FAST, false, false>(pk, total, st);
}
}  // namespace

template <int KM>
int launch_state_bwd_mfma_pack(const MfmaPack& pk, int total, bool fast, bool has_q, bool has_inj, hipStream_t st) {
  return fast ? launch_bwd_pack_flags<KM, true>(pk, total, has_q, has_inj, st)
              : launch_bwd_pack_flags<KM, false>(pk, total, has_q, has_inj, st);
}

template int launch_state_fwd_mfma_pack<256>(const MfmaPack&, int, bool, hipStream_t);
template int launch_state_bwd_mfma_pack<256>(const MfmaPack&, int, bool, bool, bool, hipStream_t);
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
