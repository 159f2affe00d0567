// Level write and residual of the block-lagged chunk model, forward and
// backward (reference _block_segment, src/gpa/attention.py:314-329, with
// _residual :190-194):
//   w = round(softmax(u(key) A^)),  rk = round(A^ w),  rv = round(w^T B^),
//   key' = round(key - eta0 rk),    value' = round(value - eta1 rv)
// for every token of a block from that block's snapshots A^ [Dk][M] and
// B^ [M][Dv].  A workgroup owns one (batch, head, block): the block's rows
// (at most 64 tokens) against its two snapshots.  The snapshots are read
// where the scans saved them (value-major chunk-start states), so nothing is
// gathered or copied; their gradients are written in the same layout, ready
// to be the scans' state gradients.  All products run on the fp32 MFMA
// (32x32x2), operands from LDS or straight from the states.
#include <hip/hip_runtime.h>

#include "mfma_tiles.h"

namespace gpa {
namespace {

constexpr int LNT = 256, LW = 4;
constexpr int LROWS = 64;  // rows (tokens) per workgroup: chunk <= 64

__host__ __device__ constexpr int pad8(int x) { return (x + 7) & ~7; }

// acc[32x32] += sum_{k<K} A(x, k) B(k, y); this lane supplies row / column
// x = y = lane % 32 and contraction indices k0 + 4 (lane / 32) + 0..3 of each
// group of 8 (the mma8 feed).  Accessors return 0 outside the matrices.
// The operands of 8 groups (64 contraction indices) are loaded before their
// MFMAs, so that the loads (often from global memory) overlap.
template <typename FA, typename FB>
__device__ __forceinline__ void tile_mma(f32x16& acc, int K, int lane, FA fa, FB fb) {
  const int x = lane & 31, kq = 4 * (lane >> 5);
  for (int k0 = 0; k0 < K; k0 += 64) {
    f32x4 a[8], b[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int k = k0 + 8 * s + kq;
      if (k0 + 8 * s < K) {
        a[s] = f32x4{fa(x, k), fa(x, k + 1), fa(x, k + 2), fa(x, k + 3)};
        b[s] = f32x4{fb(k, x), fb(k + 1, x), fb(k + 2, x), fb(k + 3, x)};
      }
    }
#pragma unroll
    for (int s = 0; s < 8; ++s)
      if (k0 + 8 * s < K) mma8(acc, a[s], b[s]);
  }
}

struct Block {
  int B, T, H, Dk, Dv, M, C, off, N;
  int b, h, n;
  bool a_first, b_first;
  const float *a_st, *b_st, *a_fs, *b_fs;

  __device__ __forceinline__ Block(const gpa_level_problem& p) {
    B = p.batch, T = p.tokens, H = p.heads, Dk = p.key_dim, Dv = p.value_dim, M = p.slots;
    C = p.chunk, off = p.offset, N = (p.offset + p.tokens + p.chunk - 1) / p.chunk;
    n = blockIdx.x, b = blockIdx.y / H, h = blockIdx.y % H;
    a_first = n == 0 && p.a_first != nullptr;
    b_first = n == 0 && p.b_first != nullptr;
    a_st = p.a_states + (((int64_t)b * H + h) * N + n) * M * Dk;  // [M][Dk]
    b_st = p.b_states + (((int64_t)b * H + h) * N + n) * Dv * M;  // [Dv][M]
    a_fs = p.a_first ? p.a_first + b * p.a_first_sb + (int64_t)h * Dk * M : nullptr;  // [Dk][M]
    b_fs = p.b_first ? p.b_first + b * p.b_first_sb + (int64_t)h * M * Dv : nullptr;  // [M][Dv]
  }
  // Token of row r, or -1 for a void row.
  __device__ __forceinline__ int token(int r) const {
    const int t = n * C + r - off;
    return (r < C && t >= 0 && t < T) ? t : -1;
  }
  __device__ __forceinline__ int64_t at(const gpa_operand& o, int t) const {
    return (int64_t)b * o.sb + (int64_t)t * o.st + (int64_t)h * o.sh;
  }
  __device__ __forceinline__ float ahat(int k, int m) const {
    if (k >= Dk || m >= M) return 0.f;
    return a_first ? a_fs[(int64_t)k * M + m] : a_st[(int64_t)m * Dk + k];
  }
  __device__ __forceinline__ float bhat(int m, int v) const {
    if (m >= M || v >= Dv) return 0.f;
    return b_first ? b_fs[(int64_t)m * Dv + v] : b_st[(int64_t)v * M + m];
  }
  // Contiguous [B,T,H,X] saved rows.
  __device__ __forceinline__ int64_t saved(int t, int width) const {
    return (((int64_t)b * T + t) * H + h) * width;
  }
};

__device__ __forceinline__ float sum4(float x) {
  x += __shfl_xor(x, 1);
  return x + __shfl_xor(x, 2);
}
__device__ __forceinline__ float max4(float x) {
  x = fmaxf(x, __shfl_xor(x, 1));
  return fmaxf(x, __shfl_xor(x, 2));
}

// Row norms of the keys (4 threads per row): den = max(||key||, 1e-6).
template <typename E>
__device__ __forceinline__ float key_den(const gpa_level_problem& p, const Block& q, int t, int part) {
  float ss = 0.f;
  if (t >= 0) {
    const E* kp = reinterpret_cast<const E*>(p.key.ptr) + q.at(p.key, t);
    for (int c = part; c < q.Dk; c += 4) {
      const float x = to_f32(kp[c]);
      ss += x * x;
    }
  }
  return fmaxf(sqrtf(sum4(ss)), 1e-6f);
}

// Slabs of the snapshots in LDS: A^ rows m0..m0+SR-1 as SL[m - m0][k]
// (pitch lsa), and B^ transposed, SL[v][m - m0] (pitch lsb).  In the usual
// case (value-major states, widths multiples of 4, a whole slab inside M) the
// slab is copied as float4s, every thread issuing all its loads before its
// stores; otherwise element by element.
constexpr int STAGE4 = 16;  // float4 copies per thread on the fast path (up to 64 KB slabs)

__device__ __forceinline__ void copy4(float* SL, const float* src, int rows, int cols, int pitch_l, int pitch_g) {
  const int per_row = cols / 4, total = rows * per_row;
  f32x4 v[STAGE4];
#pragma unroll
  for (int i = 0; i < STAGE4; ++i) {
    const int idx = threadIdx.x + i * LNT;
    if (idx < total) {
      const int r = idx / per_row, c = 4 * (idx - r * per_row);
      v[i] = *reinterpret_cast<const f32x4*>(src + (int64_t)r * pitch_g + c);
    }
  }
#pragma unroll
  for (int i = 0; i < STAGE4; ++i) {
    const int idx = threadIdx.x + i * LNT;
    if (idx < total) {
      const int r = idx / per_row, c = 4 * (idx - r * per_row);
      *reinterpret_cast<f32x4*>(SL + r * pitch_l + c) = v[i];
    }
  }
}

template <int SR>
__device__ __forceinline__ void stage_a(const Block& q, float* SL, int lsa, int m0) {
  const int nc = pad8(q.Dk);
  if (!q.a_first && q.Dk == nc && m0 + SR <= q.M && SR * nc <= 4 * STAGE4 * LNT) {
    copy4(SL, q.a_st + (int64_t)m0 * q.Dk, SR, nc, lsa, q.Dk);
    return;
  }
  for (int idx = threadIdx.x; idx < SR * nc; idx += LNT) {
    const int r = idx / nc, k = idx - r * nc;
    SL[r * lsa + k] = q.ahat(k, m0 + r);
  }
}
template <int SR>
__device__ __forceinline__ void stage_b(const Block& q, float* SL, int lsb, int m0) {
  if (!q.b_first && q.M % 4 == 0 && m0 + SR <= q.M && q.Dv * SR <= 4 * STAGE4 * LNT) {
    copy4(SL, q.b_st + m0, q.Dv, SR, lsb, q.M);
    return;
  }
  for (int idx = threadIdx.x; idx < q.Dv * SR; idx += LNT) {
    const int v = idx / SR, mm = idx - v * SR;
    SL[v * lsb + mm] = q.bhat(m0 + mm, v);
  }
}

struct LevelLds {
  int ldk, ldv, ldm, lsa, lsb, slab;
  __host__ __device__ LevelLds(int Dk, int Dv, int M, int SR) {
    ldk = pad8(Dk) + 4, ldv = pad8(Dv) + 4, ldm = pad8(M) + 4, lsa = pad8(Dk) + 4, lsb = SR + 4;
    slab = SR * lsa > Dv * lsb ? SR * lsa : Dv * lsb;
  }
  __host__ __device__ int fwd_floats() const { return LROWS * (ldk + ldm) + slab; }
  __host__ __device__ int bwd_floats() const { return LROWS * (ldk + ldv + ldm) + slab; }
};

template <typename E, int SR>
__global__ __launch_bounds__(LNT, 1) void level_fwd(gpa_level_problem p) {
  HIP_DYNAMIC_SHARED(float, lds)
  const Block q(p);
  const int Dk = q.Dk, Dv = q.Dv, M = q.M;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const LevelLds L(Dk, Dv, M, SR);
  const int ldk = L.ldk, ldm = L.ldm, lsa = L.lsa, lsb = L.lsb;
  float* KB = lds;                 // u(key), rounded        [64][ldk]
  float* S = KB + LROWS * ldk;     // logits, then w         [64][ldm]
  float* SL = S + LROWS * ldm;     // snapshot slab
  const int KT = (Dk + 31) / 32, VT = (Dv + 31) / 32;

  {  // u(key) rows, 4 threads per row
    const int row = tid >> 2, part = tid & 3, t = q.token(row);
    const float den = key_den<E>(p, q, t, part);
    const E* kp = reinterpret_cast<const E*>(p.key.ptr) + (t >= 0 ? q.at(p.key, t) : 0);
    for (int c = part; c < pad8(Dk); c += 4)
      KB[row * ldk + c] = (t >= 0 && c < Dk) ? round_as<E>(to_f32(kp[c]) / den) : 0.f;
  }
  for (int m0 = 0; m0 < M; m0 += SR) {  // logits u(key) A^, one slab of columns at a time
    __syncthreads();
    stage_a<SR>(q, SL, lsa, m0);
    __syncthreads();
    for (int t = wave; t < 2 * (SR / 32); t += LW) {
      const int rt = t & 1, ct = t >> 1;
      if (m0 + ct * 32 >= M) continue;
      f32x16 acc = {};
      tile_mma(acc, Dk, lane, [&](int x, int k) { return KB[(rt * 32 + x) * ldk + k]; },
               [&](int k, int y) { return SL[(ct * 32 + y) * lsa + k]; });
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = rt * 32 + acc_row(r, lane >> 5), col = m0 + ct * 32 + (lane & 31);
        if (col < M) S[row * ldm + col] = acc[r];
      }
    }
  }
  __syncthreads();

  {  // w = softmax, 4 threads per row; the row max and sum are saved
    const int row = tid >> 2, part = tid & 3, t = q.token(row);
    float mx = -INFINITY;
    for (int m = part; m < M; m += 4) mx = fmaxf(mx, S[row * ldm + m]);
    mx = max4(mx);
    float s = 0.f;
    for (int m = part; m < M; m += 4) s += __expf(S[row * ldm + m] - mx);
    s = sum4(s);
    if (t >= 0 && part < 2) p.stats[q.saved(t, 2) + part] = part ? s : mx;
    E* wo = reinterpret_cast<E*>(p.write.ptr) + (t >= 0 ? q.at(p.write, t) : 0);
    for (int m = part; m < pad8(M); m += 4) {
      float w = 0.f;
      if (t >= 0 && m < M) {
        w = round_as<E>(__expf(S[row * ldm + m] - mx) / s);
        wo[m] = from_f32<E>(w);
      }
      S[row * ldm + m] = w;
    }
  }

  // rk = A^ w and rv = w^T B^, summed over the slabs
  constexpr int TMAX = 2 * (GPA_LEVEL_MAX_WIDTH / 32) / LW;
  f32x16 rk[TMAX], rv[TMAX];
#pragma unroll
  for (int i = 0; i < TMAX; ++i) rk[i] = rv[i] = f32x16{};
  for (int m0 = 0; m0 < M; m0 += SR) {
    const int kc = M - m0 < SR ? M - m0 : SR;
    __syncthreads();
    stage_a<SR>(q, SL, lsa, m0);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TMAX; ++i) {
      const int t = wave + LW * i, rt = t & 1, ct = t >> 1;
      if (t < 2 * KT)
        tile_mma(rk[i], kc, lane, [&](int x, int mm) { return S[(rt * 32 + x) * ldm + m0 + mm]; },
                 [&](int mm, int y) { return ct * 32 + y < Dk ? SL[mm * lsa + ct * 32 + y] : 0.f; });
    }
    __syncthreads();
    stage_b<SR>(q, SL, lsb, m0);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TMAX; ++i) {
      const int t = wave + LW * i, rt = t & 1, ct = t >> 1;
      if (t < 2 * VT)
        tile_mma(rv[i], kc, lane, [&](int x, int mm) { return S[(rt * 32 + x) * ldm + m0 + mm]; },
                 [&](int mm, int y) { return ct * 32 + y < Dv ? SL[(ct * 32 + y) * lsb + mm] : 0.f; });
    }
  }

  const float eta0 = p.eta[2 * q.h], eta1 = p.eta[2 * q.h + 1];
#pragma unroll
  for (int i = 0; i < TMAX; ++i) {
    const int t = wave + LW * i, rt = t & 1, ct = t >> 1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = rt * 32 + acc_row(r, lane >> 5), col = ct * 32 + (lane & 31), tk = q.token(row);
      if (t < 2 * KT && col < Dk && tk >= 0) {  // key' = key - eta0 rk
        const float x = round_as<E>(rk[i][r]);
        const float key = to_f32(reinterpret_cast<const E*>(p.key.ptr)[q.at(p.key, tk) + col]);
        reinterpret_cast<E*>(p.key_out.ptr)[q.at(p.key_out, tk) + col] = from_f32<E>(round_as<E>(key - eta0 * x));
        reinterpret_cast<E*>(p.rk)[q.saved(tk, Dk) + col] = from_f32<E>(x);
      }
      if (t < 2 * VT && col < Dv && tk >= 0) {  // value' = value - eta1 rv
        const float x = round_as<E>(rv[i][r]);
        const float val = to_f32(reinterpret_cast<const E*>(p.value.ptr)[q.at(p.value, tk) + col]);
        reinterpret_cast<E*>(p.value_out.ptr)[q.at(p.value_out, tk) + col] =
            from_f32<E>(round_as<E>(val - eta1 * x));
        reinterpret_cast<E*>(p.rv)[q.saved(tk, Dv) + col] = from_f32<E>(x);
      }
    }
  }
}

template <typename E, int SR>
__global__ __launch_bounds__(LNT, 1) void level_bwd(gpa_level_problem p, gpa_level_grads g) {
  HIP_DYNAMIC_SHARED(float, lds)
  __shared__ float den_s[LROWS], mx_s[LROWS], sm_s[LROWS], dot_s[LROWS];
  __shared__ float red[LW][2];
  const Block q(p);
  const int Dk = q.Dk, Dv = q.Dv, M = q.M, H = q.H, N = q.N;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const LevelLds L(Dk, Dv, M, SR);
  const int ldk = L.ldk, ldm = L.ldm, lsa = L.lsa, lsb = L.lsb, ldx = L.ldk + L.ldv;
  float* X = lds;                // d rk | d rv, then u(key), then d u(key)   [64][ldx]
  float* Y = X + LROWS * ldx;    // w, then d w, then d logits               [64][ldm]
  float* SL = Y + LROWS * ldm;   // snapshot slab
  float* DRK = X;
  float* DRV = X + ldk;
  const int MT = (M + 31) / 32, KT = (Dk + 31) / 32, VT = (Dv + 31) / 32;
  const float eta0 = p.eta[2 * q.h], eta1 = p.eta[2 * q.h + 1];
  const E* key = reinterpret_cast<const E*>(p.key.ptr);
  float d_eta0 = 0.f, d_eta1 = 0.f;

  {  // d rk = -eta0 d key', d rv = -eta1 d value', w; row norms and softmax statistics
    const int row = tid >> 2, part = tid & 3, t = q.token(row);
    const float den = key_den<E>(p, q, t, part);
    if (part == 0) {
      den_s[row] = den;
      mx_s[row] = t >= 0 ? p.stats[q.saved(t, 2)] : 0.f;
      sm_s[row] = t >= 0 ? p.stats[q.saved(t, 2) + 1] : 1.f;
      dot_s[row] = 0.f;
    }
    const E* dko = reinterpret_cast<const E*>(g.dkey_out.ptr) + (t >= 0 ? q.at(g.dkey_out, t) : 0);
    const E* dvo = reinterpret_cast<const E*>(g.dvalue_out.ptr) + (t >= 0 ? q.at(g.dvalue_out, t) : 0);
    const E* rkp = reinterpret_cast<const E*>(p.rk) + (t >= 0 ? q.saved(t, Dk) : 0);
    const E* rvp = reinterpret_cast<const E*>(p.rv) + (t >= 0 ? q.saved(t, Dv) : 0);
    const E* w = reinterpret_cast<const E*>(p.write.ptr) + (t >= 0 ? q.at(p.write, t) : 0);
    for (int c = part; c < pad8(Dk); c += 4) {
      float d = 0.f;
      if (t >= 0 && c < Dk) {
        const float dk = to_f32(dko[c]);
        d = round_as<E>(-eta0 * dk);
        d_eta0 -= dk * to_f32(rkp[c]);
      }
      DRK[row * ldx + c] = d;
    }
    for (int c = part; c < pad8(Dv); c += 4) {
      float d = 0.f;
      if (t >= 0 && c < Dv) {
        const float dv = to_f32(dvo[c]);
        d = round_as<E>(-eta1 * dv);
        d_eta1 -= dv * to_f32(rvp[c]);
      }
      DRV[row * ldx + c] = d;
    }
    for (int m = part; m < pad8(M); m += 4) Y[row * ldm + m] = (t >= 0 && m < M) ? to_f32(w[m]) : 0.f;
  }
  __syncthreads();

  // d A^ (transposed, [M][Dk]) = w^T d rk  (completed below with d logits^T u(key))
  auto da_at = [&](int m, int k) -> float* {
    return q.a_first ? g.da_first + ((int64_t)q.b * H + q.h) * Dk * M + (int64_t)k * M + m
                     : g.da_states + (((int64_t)q.b * H + q.h) * N + q.n) * M * Dk + (int64_t)m * Dk + k;
  };
  for (int t = wave; t < MT * KT; t += LW) {
    const int mt = t % MT, kt = t / MT;
    f32x16 acc = {};
    tile_mma(acc, LROWS, lane, [&](int x, int c) { return mt * 32 + x < M ? Y[c * ldm + mt * 32 + x] : 0.f; },
             [&](int c, int y) { return kt * 32 + y < Dk ? DRK[c * ldx + kt * 32 + y] : 0.f; });
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = mt * 32 + acc_row(r, lane >> 5), k = kt * 32 + (lane & 31);
      if (m < M && k < Dk) *da_at(m, k) = acc[r];
    }
  }
  // d B^ (transposed, [Dv][M]) = d rv^T w
  for (int t = wave; t < VT * MT; t += LW) {
    const int vt = t % VT, mt = t / VT;
    f32x16 acc = {};
    tile_mma(acc, LROWS, lane,
             [&](int x, int c) { return vt * 32 + x < Dv ? DRV[c * ldx + vt * 32 + x] : 0.f; },
             [&](int c, int y) { return mt * 32 + y < M ? Y[c * ldm + mt * 32 + y] : 0.f; });
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int v = vt * 32 + acc_row(r, lane >> 5), m = mt * 32 + (lane & 31);
      if (v < Dv && m < M) {
        if (q.b_first)
          g.db_first[((int64_t)q.b * H + q.h) * M * Dv + (int64_t)m * Dv + v] = acc[r];
        else
          g.db_states[(((int64_t)q.b * H + q.h) * N + q.n) * Dv * M + (int64_t)v * M + m] = acc[r];
      }
    }
  }

  // d w = d write + d rk A^ + d rv B^T  -> Y, one slab of columns at a time
  for (int m0 = 0; m0 < M; m0 += SR) {
    __syncthreads();
    stage_b<SR>(q, SL, lsb, m0);
    __syncthreads();
    f32x16 acc = {};
    const int t = wave, rt = t & 1, ct = t >> 1;
    const bool mine = t < 2 * (SR / 32) && m0 + ct * 32 < M;
    if (mine)
      tile_mma(acc, Dv, lane, [&](int x, int v) { return DRV[(rt * 32 + x) * ldx + v]; },
               [&](int v, int y) { return v < Dv ? SL[v * lsb + ct * 32 + y] : 0.f; });
    __syncthreads();
    stage_a<SR>(q, SL, lsa, m0);
    __syncthreads();
    if (mine) {
      tile_mma(acc, Dk, lane, [&](int x, int k) { return DRK[(rt * 32 + x) * ldx + k]; },
               [&](int k, int y) { return SL[(ct * 32 + y) * lsa + k]; });
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = rt * 32 + acc_row(r, lane >> 5), m = m0 + ct * 32 + (lane & 31), tk = q.token(row);
        if (m < M) {
          float d = 0.f;
          if (tk >= 0) {
            const float dw = to_f32(reinterpret_cast<const E*>(g.dwrite.ptr)[q.at(g.dwrite, tk) + m]);
            d = round_as<E>(dw + round_as<E>(acc[r]));
          }
          Y[row * ldm + m] = d;
        }
      }
    }
  }
  __syncthreads();

  {  // u(key) -> X
    const int row = tid >> 2, part = tid & 3, t = q.token(row);
    const float den = den_s[row];
    const E* kr = key + (t >= 0 ? q.at(p.key, t) : 0);
    for (int c = part; c < pad8(Dk); c += 4)
      X[row * ldx + c] = (t >= 0 && c < Dk) ? round_as<E>(to_f32(kr[c]) / den) : 0.f;
  }

  // d logits = p (d w - <p, d w>) with p recomputed from the logits and the
  // saved row statistics: first the row dots, then d logits -> Y
  for (int pass = 0; pass < 2; ++pass) {
    for (int m0 = 0; m0 < M; m0 += SR) {
      __syncthreads();
      stage_a<SR>(q, SL, lsa, m0);
      __syncthreads();
      for (int t = wave; t < 2 * (SR / 32); t += LW) {
        const int rt = t & 1, ct = t >> 1;
        if (m0 + ct * 32 >= M) continue;
        f32x16 acc = {};
        tile_mma(acc, Dk, lane, [&](int x, int k) { return X[(rt * 32 + x) * ldx + k]; },
                 [&](int k, int y) { return SL[(ct * 32 + y) * lsa + k]; });
        float part[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = rt * 32 + acc_row(r, lane >> 5), m = m0 + ct * 32 + (lane & 31);
          const float pr = m < M ? __expf(acc[r] - mx_s[row]) / sm_s[row] : 0.f;
          const float dw = m < M ? Y[row * ldm + m] : 0.f;
          if (pass == 0) {
            part[r] = pr * dw;
          } else if (m < M) {
            Y[row * ldm + m] = pr * (dw - dot_s[row]);
          }
        }
        if (pass == 0) {
          const float tot = tile_row_sum(part, lane);  // row sum over this tile's 32 columns
          const int r = sum_index(lane);
          if ((lane & 1) == 0) atomicAdd(&dot_s[rt * 32 + acc_row(r, lane >> 5)], tot);
        }
      }
    }
  }
  __syncthreads();

  // d A^ += d logits^T u(key)  (the same tiles and lanes as above)
  for (int t = wave; t < MT * KT; t += LW) {
    const int mt = t % MT, kt = t / MT;
    f32x16 acc = {};
    tile_mma(acc, LROWS, lane, [&](int x, int c) { return mt * 32 + x < M ? Y[c * ldm + mt * 32 + x] : 0.f; },
             [&](int c, int y) { return kt * 32 + y < Dk ? X[c * ldx + kt * 32 + y] : 0.f; });
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = mt * 32 + acc_row(r, lane >> 5), k = kt * 32 + (lane & 31);
      if (m < M && k < Dk) *da_at(m, k) += acc[r];
    }
  }

  // d u(key) = d logits A^T, summed over the slabs, then -> X
  constexpr int TMAX = 2 * (GPA_LEVEL_MAX_WIDTH / 32) / LW;
  f32x16 du[TMAX];
#pragma unroll
  for (int i = 0; i < TMAX; ++i) du[i] = f32x16{};
  for (int m0 = 0; m0 < M; m0 += SR) {
    const int kc = M - m0 < SR ? M - m0 : SR;
    __syncthreads();
    stage_a<SR>(q, SL, lsa, m0);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TMAX; ++i) {
      const int t = wave + LW * i, rt = t & 1, ct = t >> 1;
      if (t < 2 * KT)
        tile_mma(du[i], kc, lane, [&](int x, int mm) { return Y[(rt * 32 + x) * ldm + m0 + mm]; },
                 [&](int mm, int y) { return ct * 32 + y < Dk ? SL[mm * lsa + ct * 32 + y] : 0.f; });
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < TMAX; ++i) {
    const int t = wave + LW * i, rt = t & 1, ct = t >> 1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = rt * 32 + acc_row(r, lane >> 5), col = ct * 32 + (lane & 31);
      if (t < 2 * KT && col < Dk) X[row * ldx + col] = round_as<E>(du[i][r]);
    }
  }
  __syncthreads();

  {  // d key = d key' + the unit-normalisation backward of d u(key)
    const int row = tid >> 2, part = tid & 3, t = q.token(row);
    const float den = den_s[row];
    float dot = 0.f;
    const E* kr = key + (t >= 0 ? q.at(p.key, t) : 0);
    if (t >= 0)
      for (int c = part; c < Dk; c += 4) dot += (to_f32(kr[c]) / den) * X[row * ldx + c];
    dot = sum4(dot);
    if (t >= 0) {
      const bool clamped = den <= 1e-6f;
      const E* dko = reinterpret_cast<const E*>(g.dkey_out.ptr) + q.at(g.dkey_out, t);
      E* dk = reinterpret_cast<E*>(g.dkey.ptr) + q.at(g.dkey, t);
      for (int c = part; c < Dk; c += 4) {
        const float u = to_f32(kr[c]) / den, duc = X[row * ldx + c];
        const float unit_bwd = clamped ? duc / den : (duc - u * dot) / den;
        dk[c] = from_f32<E>(round_as<E>(to_f32(dko[c]) + round_as<E>(unit_bwd)));
      }
    }
  }

  {  // per-block sums of d eta
    float a = d_eta0, c = d_eta1;
    for (int o = 32; o >= 1; o >>= 1) {
      a += __shfl_xor(a, o);
      c += __shfl_xor(c, o);
    }
    if (lane == 0) {
      red[wave][0] = a;
      red[wave][1] = c;
    }
    __syncthreads();
    if (tid < 2) {
      float x = 0.f;
      for (int w = 0; w < LW; ++w) x += red[w][tid];
      g.deta[(((int64_t)q.b * H + q.h) * N + q.n) * 2 + tid] = x;
    }
  }
}

int check_level(const gpa_level_problem* p) {
  if (!p) return fail(GPA_HIP_EINVAL, "level: null problem");
  if (p->batch < 1 || p->tokens < 1 || p->heads < 1) return fail(GPA_HIP_EINVAL, "level: empty shape");
  if (p->key_dim < 1 || p->key_dim > GPA_LEVEL_MAX_WIDTH || p->value_dim < 1 ||
      p->value_dim > GPA_LEVEL_MAX_WIDTH || p->slots < 1 || p->slots > GPA_LEVEL_MAX_WIDTH)
    return fail(GPA_HIP_EUNSUPPORTED, "level: key, value and slot widths must be in [1, 256]");
  if (p->chunk < 1 || p->chunk > LROWS || p->offset < 0 || p->offset >= p->chunk)
    return fail(GPA_HIP_EINVAL, "level: need 1 <= chunk <= 64 and 0 <= offset < chunk");
  if (p->dtype != GPA_DTYPE_F32 && p->dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "level: dtype");
  if (!p->key.ptr || !p->value.ptr || !p->a_states || !p->b_states || !p->eta || !p->write.ptr || !p->rk ||
      !p->rv)
    return fail(GPA_HIP_EINVAL, "level: null pointer");
  return GPA_HIP_OK;
}

constexpr size_t LDS_MAX = 160 * 1024;

// The slab height: 64 rows of the snapshots if the workgroup's LDS fits, else 32.
int slab_rows(const gpa_level_problem& p, bool backward) {
  const LevelLds big(p.key_dim, p.value_dim, p.slots, 64);
  const size_t bytes = sizeof(float) * (backward ? big.bwd_floats() : big.fwd_floats()) +
                       (backward ? 4 * LROWS * sizeof(float) + 64 : 0);
  return bytes <= LDS_MAX ? 64 : 32;
}

template <typename K>
int level_lds(K kernel, size_t bytes) {
  if (bytes > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)bytes) != hipSuccess)
    return fail(GPA_HIP_EHIP, "level: cannot raise the LDS limit");
  return GPA_HIP_OK;
}

template <typename E, int SR>
int launch_level_fwd(const gpa_level_problem& p, dim3 grid, hipStream_t stream) {
  const size_t lds = sizeof(float) * LevelLds(p.key_dim, p.value_dim, p.slots, SR).fwd_floats();
  if (int rc = level_lds(level_fwd<E, SR>, lds)) return rc;
  hipLaunchKernelGGL((level_fwd<E, SR>), grid, dim3(LNT), lds, stream, p);
  return GPA_HIP_OK;
}
template <typename E, int SR>
int launch_level_bwd(const gpa_level_problem& p, const gpa_level_grads& g, dim3 grid, hipStream_t stream) {
  const size_t lds = sizeof(float) * LevelLds(p.key_dim, p.value_dim, p.slots, SR).bwd_floats();
  if (int rc = level_lds(level_bwd<E, SR>, lds)) return rc;
  hipLaunchKernelGGL((level_bwd<E, SR>), grid, dim3(LNT), lds, stream, p, g);
  return GPA_HIP_OK;
}

}  // namespace
}  // namespace gpa

extern "C" int gpa_level_forward(const gpa_level_problem* problem, hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_level(problem)) return rc;
  if (!problem->key_out.ptr || !problem->value_out.ptr || !problem->stats)
    return fail(GPA_HIP_EINVAL, "level: null output");
  const int N = (problem->offset + problem->tokens + problem->chunk - 1) / problem->chunk;
  const dim3 grid(N, problem->batch * problem->heads);
  const bool bf = problem->dtype == GPA_DTYPE_BF16, big = slab_rows(*problem, false) == 64;
  int rc = bf ? (big ? launch_level_fwd<bf16_t, 64>(*problem, grid, stream)
                     : launch_level_fwd<bf16_t, 32>(*problem, grid, stream))
              : (big ? launch_level_fwd<float, 64>(*problem, grid, stream)
                     : launch_level_fwd<float, 32>(*problem, grid, stream));
  if (rc) return rc;
  return check_launch("gpa_level_forward");
}

extern "C" int gpa_level_backward(const gpa_level_problem* problem, const gpa_level_grads* grads,
                                  hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_level(problem)) return rc;
  if (!grads || !grads->dwrite.ptr || !grads->dkey_out.ptr || !grads->dvalue_out.ptr || !grads->dkey.ptr ||
      !grads->da_states || !grads->db_states || !grads->deta || !problem->stats ||
      (problem->a_first && !grads->da_first) || (problem->b_first && !grads->db_first))
    return fail(GPA_HIP_EINVAL, "level: null gradient buffer");
  const int N = (problem->offset + problem->tokens + problem->chunk - 1) / problem->chunk;
  const dim3 grid(N, problem->batch * problem->heads);
  const bool bf = problem->dtype == GPA_DTYPE_BF16, big = slab_rows(*problem, true) == 64;
  int rc = bf ? (big ? launch_level_bwd<bf16_t, 64>(*problem, *grads, grid, stream)
                     : launch_level_bwd<bf16_t, 32>(*problem, *grads, grid, stream))
              : (big ? launch_level_bwd<float, 64>(*problem, *grads, grid, stream)
                     : launch_level_bwd<float, 32>(*problem, *grads, grid, stream));
  if (rc) return rc;
  return check_launch("gpa_level_backward");
}
