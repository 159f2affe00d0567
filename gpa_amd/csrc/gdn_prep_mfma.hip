// Chunk preparation of the GDN scan on fp32 MFMA: one block per (chunk,
// stream), 8 waves.  Per chunk of positions t, u < 64:
//   G     in-chunk cumulative log decay (a wave scan of g)
//   Kn,Qn x/|x| rounded to the activation type, and their bf16 fragments
//   A     strictly lower b_t e^{G_t-G_u} Kn_t . Kn_u          (K Kn^T on MFMA)
//   T     (I + A)^-1: 16 x 16 diagonal blocks by forward substitution, then
//         block rows i = 1..3: T_ij = -T_ii sum_{j<=m<i} A_im T_mj
//   W     T diag(b e^G) Kn   (bf16 hi/lo fragments, or fp32 rows)
//   U     T diag(b) V        (value-major fp32)
// with the layouts of include/gpa_hip.h.  Reference: the WY form of the
// chunked gated delta rule that src/gpa/ops.py:49-85 runs per token.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "mfma_tiles.h"

namespace gpa {

constexpr int PREP_WAVES = 8, PREP_NT = 64 * PREP_WAVES;

// LDS plan (floats): one region holds Kn rows, then W (the fragment source,
// once the W product has read Kn), then the b-scaled V slices; T; A (until T
// is done); per-row scalars.  Up to 128 keys this is under 80 KB, so two
// workgroups share a compute unit.
template <int KM>
struct PrepLayout {
  static constexpr int LK = KM + 4, LT = R + 4, VC = 128, LV = VC + 4;
  static constexpr int BIG = R * LK > R * LV ? R * LK : R * LV;
  static constexpr int KN_OFF = 0, T_OFF = BIG, A_OFF = T_OFF + R * LT;
  static constexpr int BLK_OFF = A_OFF + R * LT;  // 3 x 16 x 16 block products
  static constexpr int SC_OFF = BLK_OFF + 3 * 256;
  static constexpr int TOTAL = SC_OFF + 4 * R;
  static constexpr size_t BYTES = sizeof(float) * TOTAL;
};

template <typename E, int KM, bool MF>
__global__ __launch_bounds__(PREP_NT, 1) void gdn_prep_mfma(gpa_gdn_problem p, gpa_gdn_saved sv, int nch) {
  using L = PrepLayout<KM>;
  constexpr int LK = L::LK, LT = L::LT, VC = L::VC, LV = L::LV, NW = PREP_WAVES, NTH = PREP_NT;
  constexpr int KT = KM / 32, NTW = KT >= 4 ? KT / 4 : 1;
  extern __shared__ __align__(16) float smem[];
  float* kn_s = smem + L::KN_OFF;  // [R][LK] Kn (rounded), then W [R][LK], then b V slices [R][LV]
  float* w_s = kn_s;
  float* v_s = kn_s;
  float* t_s = smem + L::T_OFF;    // [R][LT] T
  float* a_s = smem + L::A_OFF;    // [R][LT] A
  float* blk = smem + L::BLK_OFF;  // [3][16][16]
  float* gam_s = smem + L::SC_OFF;
  float* bet_s = gam_s + R;
  float* sc_s = bet_s + R;  // b e^G
  int* tok_s = reinterpret_cast<int*>(sc_s + R);

  const int n = blockIdx.x, s = blockIdx.y, b = s / p.heads, h = s % p.heads;
  const int K = p.kdim, V = p.vdim, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, hh = lane >> 5;
  const int K16 = K / 16;
  const int64_t chunk_id = (int64_t)s * nch + n;
  const bool has_q = p.q.ptr != nullptr, rows16 = MF && qk_rows_bf16(p);

  // ---- gates: G by a wave-wide inclusive scan (wave 0).
  if (wave == 0) {
    const int tok = token_at(p, n, lane), tt = tok >= 0 ? tok : 0;
    float g = scalar_load(p.g, b, h, tt), be = scalar_load(p.beta, b, h, tt);
    g = tok >= 0 ? g : 0.f;
    be = tok >= 0 ? be : 0.f;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_up(g, off);
      if (lane >= off) g += y;
    }
    gam_s[lane] = g;
    bet_s[lane] = be;
    sc_s[lane] = be * __expf(g);
    tok_s[lane] = tok;
    sv.gam[rows_off(s, n, nch, 0, 1) + lane] = g;
    sv.beta[rows_off(s, n, nch, 0, 1) + lane] = be;
  }
  // T starts as zeros (its upper blocks stay so).
  for (int i = tid; i < R * LT; i += NTH) t_s[i] = 0.f;

  // ---- normalise keys and queries: wave w owns rows w, w + 8, ...; every
  // load is issued (at a clamped address) before the first use.
  __bf16* qcol = MF && has_q ? reinterpret_cast<__bf16*>(sv.qcol) + chunk_id * frag_col_elems(K, 8) : nullptr;
  {
    constexpr int NI = KM / 64, NR = R / NW;
    const gpa_operand& qsrc = has_q ? p.q : p.k;
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
      const float dk = fmaxf(sqrtf(sum64(sk)), 1e-6f), dq = fmaxf(sqrtf(sum64(sq)), 1e-6f);
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int d = lane + 64 * i;
        const float yk = round_as<E>(xk[j][i] / dk);
        kn_s[r * LK + d] = yk;
        // (where the bf16 out and dd0 kernels read them, the Kn rows are the
        // krow fragments written below)
        if (d < K && !rows16) sv.kn[rows_off(s, n, nch, r, K) + d] = yk;
        if (has_q && d < K) {
          const float yq = round_as<E>(xq[j][i] / dq);
          if (rows16) reinterpret_cast<bf16_t*>(sv.qn)[rows_off(s, n, nch, r, K) + d] = from_f32<bf16_t>(yq);
          else sv.qn[rows_off(s, n, nch, r, K) + d] = yq;
          if (MF) {  // Qn^T fragment (d/32, r/16), lane d%32 + 32 ((r/8) % 2), element r % 8
            const int rb = d >> 5, cs = r >> 4, ln = (d & 31) + 32 * ((r >> 3) & 1);
            qcol[((rb * 4 + cs) * 64 + ln) * 8 + (r & 7)] = (__bf16)yq;
          }
        }
      }
    }
  }
  __syncthreads();

  typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
  if (MF) {
    // Kn row and column fragments (exact in bf16), one 16-byte piece per step.
    __bf16* krow = reinterpret_cast<__bf16*>(sv.krow) + chunk_id * frag_row_elems(K, 8);
    __bf16* kcol = reinterpret_cast<__bf16*>(sv.kcol) + chunk_id * frag_col_elems(K, 8);
    for (int piece = tid; piece < 2 * K16 * 64; piece += NTH) {
      const int ln = piece & 63, ks = (piece >> 6) % K16, rt = (piece >> 6) / K16;
      const float* src = kn_s + (32 * rt + (ln & 31)) * LK + 16 * ks + 8 * (ln >> 5);
      bf16x8v f;
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = (__bf16)src[e];
      *reinterpret_cast<bf16x8v*>(krow + (int64_t)piece * 8) = f;
    }
    const int RB = (K + 31) / 32;
    for (int piece = tid; piece < RB * 4 * 64; piece += NTH) {
      const int ln = piece & 63, cs = (piece >> 6) & 3, rb = piece >> 8;
      const int k = 32 * rb + (ln & 31), c0 = 16 * cs + 8 * (ln >> 5);
      bf16x8v f;
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = (__bf16)(k < K ? kn_s[(c0 + e) * LK + k] : 0.f);
      *reinterpret_cast<bf16x8v*>(kcol + (int64_t)piece * 8) = f;
    }
  }

  // ---- A = strictly lower b_t e^{G_t-G_u} Kn Kn^T: waves 0-3, one 32x32 tile each.
  if (wave < 4) {
    const int rr = wave >> 1, ru = wave & 1;
    f32x16 acc = {};
    if (std::is_same<E, bf16_t>::value) {
#pragma unroll 4
      for (int g = 0; g < KM / 16; ++g) {
        const int c0 = 16 * g + 8 * hh;
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pack8(kn_s + (32 * rr + li) * LK + c0),
                                                       pack8(kn_s + (32 * ru + li) * LK + c0), acc, 0, 0, 0);
      }
    } else {
#pragma unroll 4
      for (int g = 0; g < KM / 8; ++g) {
        const int c0 = 8 * g + 4 * hh;
        mma8(acc, ld_c(kn_s, LK, 32 * rr + li, c0), ld_c(kn_s, LK, 32 * ru + li, c0));
      }
    }
    const int u = 32 * ru + li;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = 32 * rr + acc_row(r, hh);
      a_s[t * LT + u] = (u < t) ? bet_s[t] * __expf(gam_s[t] - gam_s[u]) * acc[r] : 0.f;
    }
  }
  __syncthreads();

  // ---- T = (I + A)^-1.  Diagonal 16x16 blocks: thread c of wave 0 owns column c.
  if (tid < R) {
    const int base = 16 * (tid >> 4), c = tid & 15;
    t_s[(base + c) * LT + base + c] = 1.f;
    for (int t = c + 1; t < 16; ++t) {
      float acc = 0.f;
      for (int u = c; u < t; ++u) acc += a_s[(base + t) * LT + base + u] * t_s[(base + u) * LT + base + c];
      t_s[(base + t) * LT + base + c] = -acc;
    }
  }
  __syncthreads();
  // Block rows: X_j = sum_{j<=m<i} A_im T_mj, then T_ij = -T_ii X_j.
  for (int i = 1; i < 4; ++i) {
    for (int idx = tid; idx < i * 256; idx += NTH) {
      const int j = idx >> 8, r = (idx >> 4) & 15, c = idx & 15;
      float acc = 0.f;
      for (int m = 16 * j; m < 16 * i; ++m) acc += a_s[(16 * i + r) * LT + m] * t_s[m * LT + 16 * j + c];
      blk[idx] = acc;
    }
    __syncthreads();
    for (int idx = tid; idx < i * 256; idx += NTH) {
      const int j = idx >> 8, r = (idx >> 4) & 15, c = idx & 15;
      float acc = 0.f;
#pragma unroll
      for (int m = 0; m < 16; ++m) acc += t_s[(16 * i + r) * LT + 16 * i + m] * blk[(j << 8) + m * 16 + c];
      t_s[(16 * i + r) * LT + 16 * j + c] = -acc;
    }
    __syncthreads();
  }
  {
    float* tri = sv.tri + rows_off(s, n, nch, 0, R);
    for (int i = tid; i < R * R / 4; i += NTH) {
      const int t = i / (R / 4), c = 4 * (i % (R / 4));
      *reinterpret_cast<f32x4*>(tri + t * R + c) = *reinterpret_cast<const f32x4*>(t_s + t * LT + c);
    }
  }

  // ---- W = T diag(b e^G) Kn.  Waves below 2 KT own NTW tiles (32 rt, 32 kt).
  const bool own = wave < 2 * KT;
  const int kt = own ? (NTW == 2 ? wave : wave % KT) : 0;
  auto tile_rt = [&](int m) { return NTW == 2 ? m : (own ? wave / KT : 0); };
  f32x16 acc[NTW];
#pragma unroll
  for (int m = 0; m < NTW; ++m) acc[m] = f32x16{};
  if (own) {
#pragma unroll 4
    for (int g = 0; g < R / 8; ++g) {
      const int c0 = 8 * g + 4 * hh;
      const f32x4 bk = ld_x(kn_s, LK, 32 * kt + li, c0);
      const f32x4 sc = *reinterpret_cast<const f32x4*>(sc_s + c0);
#pragma unroll
      for (int m = 0; m < NTW; ++m) mma8(acc[m], ld_c(t_s, LT, 32 * tile_rt(m) + li, c0) * sc, bk);
    }
  }
  if (MF) __syncthreads();  // every wave has read Kn before W takes its place
  if (own) {
    const int k = 32 * kt + li;
    if (MF) {
      // W rows to LDS for the fragment writers.
#pragma unroll
      for (int m = 0; m < NTW; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) w_s[(32 * tile_rt(m) + acc_row(r, hh)) * LK + k] = acc[m][r];
    } else if (k < K) {
#pragma unroll
      for (int m = 0; m < NTW; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) sv.w[rows_off(s, n, nch, 32 * tile_rt(m) + acc_row(r, hh), K) + k] = acc[m][r];
    }
  }
  __syncthreads();
  if (MF) {
    // Row fragments: piece (t/32, k/16, lane t%32 + 32 ((k/8) % 2)); fragment f
    // = piece / 64 holds the 64 lanes' hi parts, then their lo parts.
    __bf16* wrow = reinterpret_cast<__bf16*>(sv.wrow) + chunk_id * frag_row_elems(K, 16);
    __bf16* wcol = reinterpret_cast<__bf16*>(sv.wcol) + chunk_id * frag_col_elems(K, 16);
    for (int piece = tid; piece < 2 * K16 * 64; piece += NTH) {
      const int ln = piece & 63, ks = (piece >> 6) % K16, rt = (piece >> 6) / K16;
      const float* src = w_s + (32 * rt + (ln & 31)) * LK + 16 * ks + 8 * (ln >> 5);
      bf16x8v hi, lo;
      {
        const float v[8] = {src[0], src[1], src[2], src[3], src[4], src[5], src[6], src[7]};
        split8(v, hi, lo);
      }
      __bf16* dst = wrow + (int64_t)(piece >> 6) * 1024 + ln * 8;
      *reinterpret_cast<bf16x8v*>(dst) = hi;
      *reinterpret_cast<bf16x8v*>(dst + 512) = lo;
    }
    // Column fragments: piece (k/32, t/16, lane k%32 + 32 ((t/8) % 2)), rows t..t+7,
    // planar like the row fragments.
    const int RB = (K + 31) / 32;
    for (int piece = tid; piece < RB * 4 * 64; piece += NTH) {
      const int ln = piece & 63, cs = (piece >> 6) & 3, rb = piece >> 8;
      const int k = 32 * rb + (ln & 31), c0 = 16 * cs + 8 * (ln >> 5);
      bf16x8v hi, lo;
      {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = k < K ? w_s[(c0 + e) * LK + k] : 0.f;
        split8(v, hi, lo);
      }
      __bf16* dst = wcol + (int64_t)(piece >> 6) * 1024 + ln * 8;
      *reinterpret_cast<bf16x8v*>(dst) = hi;
      *reinterpret_cast<bf16x8v*>(dst + 512) = lo;
    }
  }

  // ---- U = T diag(b) V in slices of 128 values; every wave owns one 32x32 tile.
  // Value-major on the FMA path, fragment order (ufrag_idx) on the MFMA path.
  float* um = sv.u + (MF ? ufrag_off(s, n, nch, V) : vc_off(s, n, nch, V));
  const int urt = wave >> 2, uvt = wave & 3;
  for (int v0 = 0; v0 < V; v0 += VC) {
    __syncthreads();  // W fragments (or the previous slice) are done with the region
    {
      constexpr int PER = R * VC / PREP_NT;
      float x[PER];
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int idx = tid + NTH * i, r = idx / VC, c = idx % VC, v = v0 + c;
        const int tok = tok_s[r];
        const bool ok = tok >= 0 && v < V;
        x[i] = op_load<E>(p.v, b, h, ok ? tok : 0, ok ? v : 0);
      }
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int idx = tid + NTH * i, r = idx / VC, c = idx % VC, v = v0 + c;
        const bool ok = tok_s[r] >= 0 && v < V;
        v_s[r * LV + c] = ok ? bet_s[r] * x[i] : 0.f;
      }
    }
    __syncthreads();
    f32x16 acc = {};
#pragma unroll 4
    for (int g = 0; g < R / 8; ++g) {
      const int c0 = 8 * g + 4 * hh;
      mma8(acc, ld_c(t_s, LT, 32 * urt + li, c0), ld_x(v_s, LV, 32 * uvt + li, c0));
    }
    const int v = v0 + 32 * uvt + li;
    if (MF) {
      // Whole 32-column strips, zero past V (the padded strip is read too).
      const int c = (v0 + 32 * uvt) >> 5;
      if (v0 + 32 * uvt < V) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<f32x4*>(um + ufrag_idx(c, urt, q, lane)) =
              v < V ? f32x4{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]} : f32x4{0.f, 0.f, 0.f, 0.f};
      }
    } else if (v < V) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<f32x4*>(um + (int64_t)v * R + 32 * urt + 8 * q + 4 * hh) =
            f32x4{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
    }
  }
}

template <typename E, int KM>
int launch_prep_mfma(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, bool mf, int nch, hipStream_t st) {
  const size_t lds = PrepLayout<KM>::BYTES;
  const void* fn = mf ? reinterpret_cast<const void*>(gdn_prep_mfma<E, KM, true>)
                      : reinterpret_cast<const void*>(gdn_prep_mfma<E, KM, false>);
  if (lds > 65536 &&
      hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
    return fail(GPA_HIP_EHIP, "hipFuncSetAttribute(max dynamic LDS) failed");
  const dim3 grid(nch, p.batch * p.heads), block(PREP_NT);
  if (mf)
    hipLaunchKernelGGL((gdn_prep_mfma<E, KM, true>), grid, block, lds, st, p, sv, nch);
  else
    hipLaunchKernelGGL((gdn_prep_mfma<E, KM, false>), grid, block, lds, st, p, sv, nch);
  return GPA_HIP_OK;
}

#define GPA_PREP_MFMA(E, KM) \
  template int launch_prep_mfma<E, KM>(const gpa_gdn_problem&, const gpa_gdn_saved&, bool, int, hipStream_t);
GPA_PREP_MFMA(float, 64)
GPA_PREP_MFMA(float, 128)
GPA_PREP_MFMA(float, 256)
GPA_PREP_MFMA(bf16_t, 64)
GPA_PREP_MFMA(bf16_t, 128)
GPA_PREP_MFMA(bf16_t, 256)
#undef GPA_PREP_MFMA

}  // namespace gpa
