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

  if (p.given_write) {  // the write is given: its rows -> S
    const int row = tid >> 2, part = tid & 3, t = q.token(row);
    const E* wi = reinterpret_cast<const E*>(p.write.ptr) + (t >= 0 ? q.at(p.write, t) : 0);
    for (int m = part; m < pad8(M); m += 4) S[row * ldm + m] = (t >= 0 && m < M) ? to_f32(wi[m]) : 0.f;
  } else {
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
  const bool given = p.given_write != 0;  // the write is an input: its gradient ends at d w
  float d_eta0 = 0.f, d_eta1 = 0.f;

  {  // d rk = -eta0 d key', d rv = -eta1 d value', w; row norms and softmax statistics
    const int row = tid >> 2, part = tid & 3, t = q.token(row);
    const float den = given ? 1.f : key_den<E>(p, q, t, part);
    if (part == 0) {
      den_s[row] = den;
      mx_s[row] = t >= 0 && !given ? p.stats[q.saved(t, 2)] : 0.f;
      sm_s[row] = t >= 0 && !given ? p.stats[q.saved(t, 2) + 1] : 1.f;
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
            const float dw = g.dwrite.ptr ? to_f32(reinterpret_cast<const E*>(g.dwrite.ptr)[q.at(g.dwrite, tk) + m])
                                          : 0.f;
            d = round_as<E>(dw + round_as<E>(acc[r]));
            if (given) reinterpret_cast<E*>(g.dwrite_given.ptr)[q.at(g.dwrite_given, tk) + m] = from_f32<E>(d);
          }
          Y[row * ldm + m] = d;
        }
      }
    }
  }
  __syncthreads();

  if (!given) {  // the write's own backward: softmax, u(key) A^ and the unit normalisation
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

// ---------------------------------------------------------------------------
// bf16 activations: the same step on the bf16 MFMA (32x32x16).  u(key), the
// write w and the reconstructions' incoming gradients are exact in bf16 (the
// reference rounds them to the activation type); the fp32 snapshots and
// gradients are split into bf16 hi + lo, each product taking hi*hi + hi*lo +
// lo*hi (the hi*lo terms vanish against an exact operand).  Snapshot
// fragments are read straight from global memory (eight contraction indices
// per lane: 32 contiguous bytes where the layout allows, else eight
// coalesced scalars), so nothing but the block's rows is staged in LDS and
// two or three workgroups share a CU.  Row phases run one wave per row with
// the lanes along the row.

__host__ __device__ constexpr int pad16(int x) { return (x + 15) & ~15; }
__host__ __device__ constexpr int pad32(int x) { return (x + 31) & ~31; }

struct Lds16 {
  int ldu, ldw, lde;       // bf16 pitch of u(key) and w rows, float pitch of the fp32 row buffer
  int u_off, w_off, e_off;  // byte offsets
  int bytes;
  __host__ __device__ Lds16(int Dk, int Dv, int M) {
    ldu = pad16(Dk) + 8;
    ldw = pad16(M) + 8;
    int wide = pad32(M) > pad32(Dk) ? pad32(M) : pad32(Dk);
    wide = wide > pad32(Dv) ? wide : pad32(Dv);
    lde = wide + 4;
    u_off = 0;
    w_off = u_off + LROWS * ldu * 2;
    e_off = w_off + LROWS * ldw * 2;
    bytes = e_off + LROWS * lde * 4;
  }
};

// A snapshot column seen along its contraction axis: element i of the column
// is base[i * st], i < count; `ok` is false for a padding column.
struct Col {
  const float* base;
  int st, count;
  bool ok;
};

// Eight consecutive elements first .. first+7 of a column, loads only:
// indices are clamped to the column, and mask8 zeroes what lies past `count`
// or in a padding column once the loads of a group are all issued (a mask
// next to its load would make the wave wait for each load in turn).  With
// FAST (count a multiple of 16) and a unit stride they are two 16-byte
// loads; the stride is one per operand, so the branch is uniform.
template <bool FAST>
__device__ __forceinline__ void raw8(const Col& c, int first, float (&v)[8]) {
  const int st = __builtin_amdgcn_readfirstlane(c.st);
  if (FAST && st == 1) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(c.base + first);
    const f32x4 b = *reinterpret_cast<const f32x4*>(c.base + first + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int i = first + e < c.count ? first + e : c.count - 1;
      v[e] = c.base[i * st];
    }
  }
}
__device__ __forceinline__ void mask8(const Col& c, int first, float (&v)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (c.ok && first + e < c.count) ? v[e] : 0.f;
}


__device__ __forceinline__ f32x16 mfma16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Snapshot columns (the out-of-range column index is clamped for the loads).
// A^ along k, column m (a slot): A^[.][m].
__device__ __forceinline__ Col ahat_k(const Block& q, int m) {
  const int mc = m < q.M ? m : q.M - 1;
  return q.a_first ? Col{q.a_fs + mc, q.M, q.Dk, m < q.M} : Col{q.a_st + (int64_t)mc * q.Dk, 1, q.Dk, m < q.M};
}
// A^ along m, column k: A^[k][.].
__device__ __forceinline__ Col ahat_m(const Block& q, int k) {
  const int kc = k < q.Dk ? k : q.Dk - 1;
  return q.a_first ? Col{q.a_fs + (int64_t)kc * q.M, 1, q.M, k < q.Dk} : Col{q.a_st + kc, q.Dk, q.M, k < q.Dk};
}
// B^ along m, column v: B^[.][v].
__device__ __forceinline__ Col bhat_m(const Block& q, int v) {
  const int vc = v < q.Dv ? v : q.Dv - 1;
  return q.b_first ? Col{q.b_fs + vc, q.Dv, q.M, v < q.Dv} : Col{q.b_st + (int64_t)vc * q.M, 1, q.M, v < q.Dv};
}

// B^ along v, column m: B^[m][.].
__device__ __forceinline__ Col bhat_v(const Block& q, int m) {
  const int mc = m < q.M ? m : q.M - 1;
  return q.b_first ? Col{q.b_fs + (int64_t)mc * q.Dv, 1, q.Dv, m < q.M} : Col{q.b_st + mc, q.M, q.Dv, m < q.M};
}

// acc[rt] += A_rt B (rt = 0, 1: the block's two 32-row tiles) over `steps`
// 16-wide contraction steps, B split into hi / lo; each B fragment is loaded
// once for both row tiles, and the fragments of FGROUP steps are loaded
// before their MFMAs so that their global loads overlap.  A fragments come
// from LDS.
constexpr int FGROUP = 8;
template <bool FAST, typename LA>
__device__ __forceinline__ void tile2_split_b(f32x16 (&acc)[2], int steps, const Col& col, int sub, LA&& frag_a) {
  f32x16 c[4] = {};
#pragma unroll 1
  for (int s0 = 0; s0 < steps; s0 += FGROUP) {
    float v[FGROUP][8];
#pragma unroll
    for (int j = 0; j < FGROUP; ++j) raw8<FAST>(col, 16 * (s0 + j < steps ? s0 + j : steps - 1) + sub, v[j]);
#pragma unroll
    for (int j = 0; j < FGROUP; ++j)
      if (s0 + j < steps) {
        mask8(col, 16 * (s0 + j) + sub, v[j]);
        bf16x8 hi, lo;
        split8(v[j], hi, lo);
        const bf16x8 a0 = frag_a(0, s0 + j), a1 = frag_a(1, s0 + j);
        c[0] = mfma16(a0, hi, c[0]);
        c[2] = mfma16(a1, hi, c[2]);
        c[1] = mfma16(a0, lo, c[1]);
        c[3] = mfma16(a1, lo, c[3]);
      }
  }
  acc[0] = c[0] + c[1];
  acc[1] = c[2] + c[3];
}

// Row phases with whole rows per 32 lanes: thread -> (row, columns 8 c32 ..
// 8 c32 + 7), 8 rows per pass of the workgroup, 8 passes; every global load
// of a thread is issued before its first use.  Needs widths that are
// multiples of 8 and at most 256.
constexpr int RPASS = LROWS / (LNT / 32);  // passes of 8 rows

__device__ __forceinline__ float sum32(float x) {
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) x += __shfl_xor(x, m, 32);
  return x;
}
__device__ __forceinline__ float max32(float x) {
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m, 32));
  return x;
}

__device__ __forceinline__ void bf8_to_f32(const uint4& u, float (&x)[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = __uint_as_float(w[i] << 16);
    x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ uint4 f32_to_bf8(const float (&x)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = (uint32_t)f32_to_bf16(x[2 * i]).bits | ((uint32_t)f32_to_bf16(x[2 * i + 1]).bits << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

template <bool FAST>
__global__ __launch_bounds__(LNT, 2) void level_fwd16(gpa_level_problem p) {
  HIP_DYNAMIC_SHARED(float, lds_f)
  unsigned char* lds = reinterpret_cast<unsigned char*>(lds_f);
  const Block q(p);
  const int Dk = q.Dk, Dv = q.Dv, M = q.M;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 31, hh = lane >> 5;
  const Lds16 L(Dk, Dv, M);
  __bf16* U = reinterpret_cast<__bf16*>(lds + L.u_off);  // u(key) [64][ldu]
  __bf16* W = reinterpret_cast<__bf16*>(lds + L.w_off);  // w [64][ldw]
  float* E = reinterpret_cast<float*>(lds + L.e_off);    // logits, then rk / rv [64][lde]
  const int ldu = L.ldu, ldw = L.ldw, lde = L.lde;
  const bf16_t* key = reinterpret_cast<const bf16_t*>(p.key.ptr);
  const int M16 = pad16(M) / 16;

  if (p.given_write) {  // the write is given: its rows -> W
    if (FAST) {
      const int c = 8 * (tid & 31), r0 = tid >> 5;
      if (c < M)
#pragma unroll
        for (int i = 0; i < RPASS; ++i) {
          const int r = r0 + 8 * i, t = q.token(r);
          *reinterpret_cast<uint4*>(&W[r * ldw + c]) =
              t >= 0 ? *reinterpret_cast<const uint4*>(reinterpret_cast<const bf16_t*>(p.write.ptr) + q.at(p.write, t) + c)
                     : make_uint4(0, 0, 0, 0);
        }
    } else
    for (int r = wave; r < LROWS; r += LW) {
      const int t = q.token(r);
      const bf16_t* wi = reinterpret_cast<const bf16_t*>(p.write.ptr) + (t >= 0 ? q.at(p.write, t) : 0);
      for (int m = lane; m < ldw; m += 64) W[r * ldw + m] = (__bf16)((t >= 0 && m < M) ? to_f32(wi[m]) : 0.f);
    }
  } else {
  // u(key)
  if (FAST) {
    const int c32 = tid & 31, c = 8 * c32, r0 = tid >> 5;
    const bool on = c < Dk;
    uint4 raw[RPASS];
#pragma unroll
    for (int i = 0; i < RPASS; ++i) {
      const int t = q.token(r0 + 8 * i);
      raw[i] = (on && t >= 0) ? *reinterpret_cast<const uint4*>(key + q.at(p.key, t) + c) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < RPASS; ++i) {
      float x[8];
      bf8_to_f32(raw[i], x);
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
      const float den = fmaxf(sqrtf(sum32(ss)), 1e-6f);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = x[e] / den;
      if (on) *reinterpret_cast<uint4*>(&U[(r0 + 8 * i) * ldu + c]) = f32_to_bf8(x);
    }
  } else
  for (int r = wave; r < LROWS; r += LW) {
    const int t = q.token(r);
    float x[GPA_LEVEL_MAX_WIDTH / 64];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < GPA_LEVEL_MAX_WIDTH / 64; ++i) {
      const int c = lane + 64 * i;
      x[i] = (t >= 0 && c < Dk) ? to_f32(key[q.at(p.key, t) + c]) : 0.f;
      ss += x[i] * x[i];
    }
    const float den = fmaxf(sqrtf(sum64(ss)), 1e-6f);
#pragma unroll
    for (int i = 0; i < GPA_LEVEL_MAX_WIDTH / 64; ++i) {
      const int c = lane + 64 * i;
      if (c < ldu) U[r * ldu + c] = (__bf16)(x[i] / den);  // exact: bf16 rounding of the unit key
    }
  }
  __syncthreads();

  // logits = u(key) A^ -> E
  const int K16 = pad16(Dk) / 16, MT = pad32(M) / 32;
#pragma unroll 1
  for (int mt = wave; mt < MT; mt += LW) {
    const int m = 32 * mt + li;
    f32x16 acc[2];
    const Col col = ahat_k(q, m);
    tile2_split_b<FAST>(
        acc, K16, col, 8 * hh,
        [&](int rt, int ks) { return *reinterpret_cast<const bf16x8*>(&U[(32 * rt + li) * ldu + 16 * ks + 8 * hh]); });
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int r = 0; r < 16; ++r) E[(32 * rt + acc_row(r, hh)) * lde + m] = acc[rt][r];
  }
  __syncthreads();

  // w = softmax; the row max and sum are saved.
  if (FAST) {
    const int c32 = tid & 31, c = 8 * c32, r0 = tid >> 5;
    const bool on = c < M;
#pragma unroll 2
    for (int i = 0; i < RPASS; ++i) {
      const int r = r0 + 8 * i, t = q.token(r);
      float x[8];
      float mx = -INFINITY;
      if (on) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(&E[r * lde + c]);
        const f32x4 b = *reinterpret_cast<const f32x4*>(&E[r * lde + c + 4]);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
#pragma unroll
        for (int e = 0; e < 8; ++e) mx = fmaxf(mx, x[e]);
      }
      mx = max32(mx);
      float sm = 0.f;
      if (on)
#pragma unroll
        for (int e = 0; e < 8; ++e) sm += __expf(x[e] - mx);
      sm = sum32(sm);
      if (t >= 0 && c32 < 2) p.stats[q.saved(t, 2) + c32] = c32 ? sm : mx;
      if (on) {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = t >= 0 ? round_as<bf16_t>(__expf(x[e] - mx) / sm) : 0.f;
        const uint4 w8 = f32_to_bf8(x);
        *reinterpret_cast<uint4*>(&W[r * ldw + c]) = w8;
        if (t >= 0) *reinterpret_cast<uint4*>(reinterpret_cast<bf16_t*>(p.write.ptr) + q.at(p.write, t) + c) = w8;
      }
    }
  } else
  for (int r = wave; r < LROWS; r += LW) {
    const int t = q.token(r);
    float x[GPA_LEVEL_MAX_WIDTH / 64];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < GPA_LEVEL_MAX_WIDTH / 64; ++i) {
      const int m = lane + 64 * i;
      x[i] = m < M ? E[r * lde + m] : -INFINITY;
      mx = fmaxf(mx, x[i]);
    }
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    float sm = 0.f;
#pragma unroll
    for (int i = 0; i < GPA_LEVEL_MAX_WIDTH / 64; ++i) sm += lane + 64 * i < M ? __expf(x[i] - mx) : 0.f;
    sm = sum64(sm);
    if (t >= 0 && lane < 2) p.stats[q.saved(t, 2) + lane] = lane ? sm : mx;
    bf16_t* wo = reinterpret_cast<bf16_t*>(p.write.ptr) + (t >= 0 ? q.at(p.write, t) : 0);
#pragma unroll
    for (int i = 0; i < GPA_LEVEL_MAX_WIDTH / 64; ++i) {
      const int m = lane + 64 * i;
      float w = 0.f;
      if (t >= 0 && m < M) {
        w = round_as<bf16_t>(__expf(x[i] - mx) / sm);
        wo[m] = from_f32<bf16_t>(w);
      }
      if (m < ldw) W[r * ldw + m] = (__bf16)w;
    }
  }
  }
  __syncthreads();

  // rk = A^ w (then key' = key - eta0 rk) and rv = w^T B^ (then value' = value - eta1 rv):
  // tiles -> E, then a wave per row writes the rounded results.
  const float eta0 = p.eta[2 * q.h], eta1 = p.eta[2 * q.h + 1];
  for (int part = 0; part < 2; ++part) {
    const int D = part ? Dv : Dk, DT = pad32(D) / 32;
#pragma unroll 1
    for (int dt = wave; dt < DT; dt += LW) {
      const int c = 32 * dt + li;
      f32x16 acc[2];
      const Col col = part ? bhat_m(q, c) : ahat_m(q, c);
      tile2_split_b<FAST>(
          acc, M16, col, 8 * hh,
          [&](int rt, int ms) {
            return *reinterpret_cast<const bf16x8*>(&W[(32 * rt + li) * ldw + 16 * ms + 8 * hh]);
          });
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int r = 0; r < 16; ++r) E[(32 * rt + acc_row(r, hh)) * lde + c] = acc[rt][r];
    }
    __syncthreads();
    const gpa_operand& src = part ? p.value : p.key;
    const gpa_operand& dst = part ? p.value_out : p.key_out;
    bf16_t* saved = reinterpret_cast<bf16_t*>(part ? p.rv : p.rk);
    const float eta = part ? eta1 : eta0;
    if (FAST) {
      const int c32 = tid & 31, c = 8 * c32, r0 = tid >> 5;
      const bool on = c < D;
      uint4 raw[RPASS];
#pragma unroll
      for (int i = 0; i < RPASS; ++i) {
        const int t = q.token(r0 + 8 * i);
        raw[i] = (on && t >= 0) ? *reinterpret_cast<const uint4*>(reinterpret_cast<const bf16_t*>(src.ptr) +
                                                                   q.at(src, t) + c)
                                : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < RPASS; ++i) {
        const int r = r0 + 8 * i, t = q.token(r);
        if (!on || t < 0) continue;
        float x[8], rc[8];
        bf8_to_f32(raw[i], x);
        const f32x4 a = *reinterpret_cast<const f32x4*>(&E[r * lde + c]);
        const f32x4 b = *reinterpret_cast<const f32x4*>(&E[r * lde + c + 4]);
        rc[0] = a.x; rc[1] = a.y; rc[2] = a.z; rc[3] = a.w; rc[4] = b.x; rc[5] = b.y; rc[6] = b.z; rc[7] = b.w;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          rc[e] = round_as<bf16_t>(rc[e]);
          x[e] = x[e] - eta * rc[e];
        }
        *reinterpret_cast<uint4*>(reinterpret_cast<bf16_t*>(dst.ptr) + q.at(dst, t) + c) = f32_to_bf8(x);
        *reinterpret_cast<uint4*>(saved + q.saved(t, D) + c) = f32_to_bf8(rc);
      }
    } else
    for (int r = wave; r < LROWS; r += LW) {
      const int t = q.token(r);
      if (t < 0) continue;
      const bf16_t* x = reinterpret_cast<const bf16_t*>(src.ptr) + q.at(src, t);
      bf16_t* y = reinterpret_cast<bf16_t*>(dst.ptr) + q.at(dst, t);
      bf16_t* sv = saved + q.saved(t, D);
      for (int c = lane; c < D; c += 64) {
        const float rc = round_as<bf16_t>(E[r * lde + c]);
        y[c] = from_f32<bf16_t>(round_as<bf16_t>(to_f32(x[c]) - eta * rc));
        sv[c] = from_f32<bf16_t>(rc);
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// The backward for bf16 activations on bf16 MFMA, for aligned widths (all
// multiples of 16, 16-byte aligned rows); other shapes keep level_bwd.
// 8 waves.  Per block (rows t, slots m, keys k, values v):
//   drk = round(-eta0 dkey'), drv = round(-eta1 dvalue')           (exact bf16)
//   dB^T = drv^T w                                                 -> db
//   dw   = round(dwrite + round(drk A^^T... + drv B^^T))  (drk A^ + drv B^T)
//   p    = softmax(u A^) from the saved row max and sum
//   dl   = p (dw - <p, dw>)
//   dA^T = w^T drk + dl^T u                                        -> da
//   du   = dl A^T;  dkey = round(dkey' + round(unit backward of round(du)))
// Products contracting over the block's rows read token-contiguous LDS
// copies (w^T, drk^T, drv^T, u^T, dl^T), written with the lanes along the
// rows; the one product contracting over slots (du) gathers its dl rows from
// dl^T.  Snapshot fragments come from global memory as in the forward.
constexpr int BW = 8, BNT = 64 * BW;  // waves, threads
constexpr int TP = LROWS + 8;         // bf16 pitch of token-contiguous rows

struct Lds16b {
  int wt, drkt, ut, drvt, dlt_hi, dlt_lo, du, bytes;  // byte offsets
  int lde;                                            // float pitch of du rows
  __host__ __device__ Lds16b(int Dk, int Dv, int M) {
    const int x = LROWS > 0 ? 2 * TP : 0;             // bytes per token-contiguous row
    wt = 0;
    drkt = wt + M * x;
    ut = drkt + Dk * x;
    dlt_hi = ut + Dk * x;
    dlt_lo = dlt_hi + M * x;
    drvt = dlt_hi;                                    // dead before dl^T is written
    lde = Dk + 4;
    const int need_du = LROWS * lde * 4, need_drvt = Dv * x;
    bytes = dlt_lo + M * x;
    if (dlt_hi + need_drvt > bytes) bytes = dlt_hi + need_drvt;
    // du replaces w^T .. u^T (dead by then) when it fits below dl^T, which is
    // still being read while du is written; else it goes after everything.
    du = need_du <= dlt_hi ? 0 : bytes;
    if (du) bytes += need_du;
  }
};

template <int TW>  // (row tile, slot tile) pairs per wave in the dw / logits phase: 2 M / 32 / BW
__global__ __launch_bounds__(BNT, 1) void level_bwd16(gpa_level_problem p, gpa_level_grads g) {
  HIP_DYNAMIC_SHARED(float, lds_f)
  unsigned char* lds = reinterpret_cast<unsigned char*>(lds_f);
  __shared__ float den_s[LROWS], mx_s[LROWS], sm_s[LROWS], dot_s[LROWS];
  __shared__ float red[BW][2];
  const Block q(p);
  const int Dk = q.Dk, Dv = q.Dv, M = q.M, H = q.H, N = q.N;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 31, hh = lane >> 5;
  const Lds16b L(Dk, Dv, M);
  __bf16* WT = reinterpret_cast<__bf16*>(lds + L.wt);     // w^T     [M][TP]
  __bf16* DRKT = reinterpret_cast<__bf16*>(lds + L.drkt); // drk^T   [Dk][TP]
  __bf16* UT = reinterpret_cast<__bf16*>(lds + L.ut);     // u^T     [Dk][TP]
  __bf16* DRVT = reinterpret_cast<__bf16*>(lds + L.drvt); // drv^T   [Dv][TP]
  __bf16* DLH = reinterpret_cast<__bf16*>(lds + L.dlt_hi); // dl^T hi [M][TP]
  __bf16* DLL = reinterpret_cast<__bf16*>(lds + L.dlt_lo); // dl^T lo
  float* DU = reinterpret_cast<float*>(lds + L.du);        // du      [64][lde]
  const float eta0 = p.eta[2 * q.h], eta1 = p.eta[2 * q.h + 1];
  const bf16_t* key = reinterpret_cast<const bf16_t*>(p.key.ptr);
  const int MT = M / 32, KT = Dk / 32, VT = Dv / 32, K16 = Dk / 16, V16 = Dv / 16, M16 = M / 16;
  const bool given = p.given_write != 0;  // the write is an input: its gradient ends at dw

  // ---- rows: norms of the keys (16 rows per pass, 32 lanes per row) and the
  // saved softmax statistics.
  if (!given) {
    const int c = 8 * (tid & 31), r0 = tid >> 5;
    uint4 raw[LROWS / 16];
#pragma unroll
    for (int i = 0; i < LROWS / 16; ++i) {
      const int t = q.token(r0 + 16 * i);
      raw[i] = (c < Dk && t >= 0) ? *reinterpret_cast<const uint4*>(key + q.at(p.key, t) + c) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < LROWS / 16; ++i) {
      float x[8];
      bf8_to_f32(raw[i], x);
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
      ss = sum32(ss);
      const int r = r0 + 16 * i, t = q.token(r);
      if ((tid & 31) == 0) {
        den_s[r] = fmaxf(sqrtf(ss), 1e-6f);
        mx_s[r] = t >= 0 ? p.stats[q.saved(t, 2)] : 0.f;
        sm_s[r] = t >= 0 ? p.stats[q.saved(t, 2) + 1] : 1.f;
        dot_s[r] = 0.f;
      }
    }
  }
  __syncthreads();

  // ---- token-contiguous copies: lane = row, wave = group of 8 columns.
  float d_eta0 = 0.f, d_eta1 = 0.f;
  {
    const int t = q.token(lane);
    auto load8 = [&](const gpa_operand& o, int c) {
      return t >= 0 ? *reinterpret_cast<const uint4*>(reinterpret_cast<const bf16_t*>(o.ptr) + q.at(o, t) + c)
                    : make_uint4(0, 0, 0, 0);
    };
    auto saved8 = [&](const void* base, int D, int c) {
      return t >= 0 ? *reinterpret_cast<const uint4*>(reinterpret_cast<const bf16_t*>(base) + q.saved(t, D) + c)
                    : make_uint4(0, 0, 0, 0);
    };
    auto put_t = [&](__bf16* dst, int c, const float (&x)[8]) {
#pragma unroll
      for (int e = 0; e < 8; ++e) dst[(c + e) * TP + lane] = (__bf16)x[e];
    };
    for (int c = 8 * wave; c < M; c += 8 * BW) {  // w^T
      float x[8];
      bf8_to_f32(load8(p.write, c), x);
      put_t(WT, c, x);
    }
    for (int c = 8 * wave; c < Dk; c += 8 * BW) {  // drk^T, u^T, d eta0
      const uint4 a = load8(g.dkey_out, c), b = saved8(p.rk, Dk, c);
      float d[8], r[8];
      bf8_to_f32(a, d);
      bf8_to_f32(b, r);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        d_eta0 -= d[e] * r[e];
        d[e] = round_as<bf16_t>(-eta0 * d[e]);
      }
      put_t(DRKT, c, d);
      if (!given) {
        float x[8];
        bf8_to_f32(load8(p.key, c), x);
        const float den = den_s[lane];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = x[e] / den;
        put_t(UT, c, x);
      }
    }
    for (int c = 8 * wave; c < Dv; c += 8 * BW) {  // drv^T, d eta1
      const uint4 a = load8(g.dvalue_out, c), b = saved8(p.rv, Dv, c);
      float d[8], r[8];
      bf8_to_f32(a, d);
      bf8_to_f32(b, r);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        d_eta1 -= d[e] * r[e];
        d[e] = round_as<bf16_t>(-eta1 * d[e]);
      }
      put_t(DRVT, c, d);
    }
  }
  __syncthreads();

  auto frag_t = [&](const __bf16* X, int row, int ts) {  // 8 tokens of row `row` of a token-contiguous copy
    return *reinterpret_cast<const bf16x8*>(&X[row * TP + 16 * ts + 8 * hh]);
  };

  // ---- dB^T[v][m] = sum_t drv[t][v] w[t][m]  -> db
  for (int i = wave; i < VT * MT; i += BW) {
    const int vt = i % VT, mt = i / VT;
    f32x16 acc = {};
#pragma unroll
    for (int ts = 0; ts < LROWS / 16; ++ts)
      acc = mfma16(frag_t(DRVT, 32 * vt + li, ts), frag_t(WT, 32 * mt + li, ts), acc);
    const int m = 32 * mt + li;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int v = 32 * vt + acc_row(r, hh);
      if (q.b_first) g.db_first[((int64_t)q.b * H + q.h) * M * Dv + (int64_t)m * Dv + v] = acc[r];
      else g.db_states[(((int64_t)q.b * H + q.h) * N + q.n) * Dv * M + (int64_t)v * M + m] = acc[r];
    }
  }

  // ---- dw and the recomputed logits per (row tile i & 1, slot tile i >> 1):
  // p and dw of the tile, in accumulator layout.
  auto dw_logits = [&](int i, float (&pk)[16], float (&dk)[16]) {
    const int rt = i & 1, mt = i >> 1;
    const int m = 32 * mt + li, row = 32 * rt + li, trow = q.token(row);
    // dwrite of the tile's elements, loaded first so that it arrives meanwhile.
    float dwr[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int tk = q.token(32 * rt + acc_row(r, hh));  // void rows: token 0, masked at use
      dwr[r] = g.dwrite.ptr
                   ? to_f32(reinterpret_cast<const bf16_t*>(g.dwrite.ptr)[q.at(g.dwrite, tk >= 0 ? tk : 0) + m])
                   : 0.f;
    }
    // A fragments from global: drk and u (contraction k), drv (contraction v).
    const bf16_t* dkr = reinterpret_cast<const bf16_t*>(g.dkey_out.ptr) + (trow >= 0 ? q.at(g.dkey_out, trow) : 0);
    const bf16_t* dvr = reinterpret_cast<const bf16_t*>(g.dvalue_out.ptr) + (trow >= 0 ? q.at(g.dvalue_out, trow) : 0);
    const bf16_t* kr = key + (trow >= 0 ? q.at(p.key, trow) : 0);
    const float den = den_s[row];
    auto a_frag = [&](const uint4& raw, float scale, bool unit) {
      float x[8];
      bf8_to_f32(raw, x);
      bf16x8 f;
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = (__bf16)(unit ? x[e] / den : round_as<bf16_t>(scale * x[e]));
      return f;
    };
    // The key-side (A^, contraction k) and value-side (B^^T, contraction v)
    // products run in one loop, so the loads of both are in flight together.
    f32x16 cw[2] = {}, cl[2] = {};
    const Col ak = ahat_k(q, m), bv = bhat_v(q, m);
    constexpr int G = 4;
    const int S16 = K16 > V16 ? K16 : V16;
#pragma unroll 1
    for (int s0 = 0; s0 < S16; s0 += G) {
      float va[G][8], vb[G][8];
      uint4 rd[G], rk[G], rv[G];
#pragma unroll
      for (int jj = 0; jj < G; ++jj) {
        const int c0 = 16 * (s0 + jj) + 8 * hh;
        raw8<true>(ak, s0 + jj < K16 ? c0 : 16 * (K16 - 1) + 8 * hh, va[jj]);
        raw8<true>(bv, s0 + jj < V16 ? c0 : 16 * (V16 - 1) + 8 * hh, vb[jj]);
        if (s0 + jj < K16) {
          rd[jj] = trow >= 0 ? *reinterpret_cast<const uint4*>(dkr + c0) : make_uint4(0, 0, 0, 0);
          rk[jj] = trow >= 0 && !given ? *reinterpret_cast<const uint4*>(kr + c0) : make_uint4(0, 0, 0, 0);
        }
        if (s0 + jj < V16) {
          rv[jj] = trow >= 0 ? *reinterpret_cast<const uint4*>(dvr + c0) : make_uint4(0, 0, 0, 0);
        }
      }
#pragma unroll
      for (int jj = 0; jj < G; ++jj) {
        if (s0 + jj < K16) {
          mask8(ak, 16 * (s0 + jj) + 8 * hh, va[jj]);
          bf16x8 bh, bl;
          split8(va[jj], bh, bl);
          const bf16x8 ad = a_frag(rd[jj], -eta0, false);
          cw[0] = mfma16(ad, bh, cw[0]);
          cw[1] = mfma16(ad, bl, cw[1]);
          if (!given) {
            const bf16x8 au = a_frag(rk[jj], 1.f, true);
            cl[0] = mfma16(au, bh, cl[0]);
            cl[1] = mfma16(au, bl, cl[1]);
          }
        }
        if (s0 + jj < V16) {
          mask8(bv, 16 * (s0 + jj) + 8 * hh, vb[jj]);
          bf16x8 bh, bl;
          split8(vb[jj], bh, bl);
          const bf16x8 ad = a_frag(rv[jj], -eta1, false);
          cw[0] = mfma16(ad, bh, cw[0]);
          cw[1] = mfma16(ad, bl, cw[1]);
        }
      }
    }
    const f32x16 dwa = cw[0] + cw[1], lga = cl[0] + cl[1];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = 32 * rt + acc_row(r, hh), tk = q.token(t);
      dk[r] = tk >= 0 ? round_as<bf16_t>(dwr[r] + round_as<bf16_t>(dwa[r])) : 0.f;
      pk[r] = given ? 0.f : __expf(lga[r] - mx_s[t]) / sm_s[t];
    }
  };
  auto add_dot = [&](int i, const float (&pk)[16], const float (&dk)[16]) {
    float part[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) part[r] = pk[r] * dk[r];
    const float tot = tile_row_sum(part, lane);
    if ((lane & 1) == 0) atomicAdd(&dot_s[32 * (i & 1) + acc_row(sum_index(lane), hh)], tot);
  };
  auto put_dl = [&](int i, const float (&pk)[16], const float (&dk)[16]) {  // dl = p (dw - dot) -> dl^T
    const int rt = i & 1, m = 32 * (i >> 1) + li;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = 32 * rt + acc_row(r, hh);
      const float x = pk[r] * (dk[r] - dot_s[t]);
      const __bf16 hi = (__bf16)x;
      DLH[m * TP + t] = hi;
      DLL[m * TP + t] = (__bf16)(x - (float)hi);
    }
  };
  if (given) {  // dw is the given write's gradient
#pragma unroll 1
    for (int i = wave; i < 2 * MT; i += BW) {
      float pk[16], dk[16];
      dw_logits(i, pk, dk);
      const int m = 32 * (i >> 1) + li;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int tk = q.token(32 * (i & 1) + acc_row(r, hh));
        if (tk >= 0)
          reinterpret_cast<bf16_t*>(g.dwrite_given.ptr)[q.at(g.dwrite_given, tk) + m] = from_f32<bf16_t>(dk[r]);
      }
    }
  } else if (TW == 1) {  // one tile per wave: p and dw stay in registers across the row-dot barrier
    const int i = wave;
    float pk[16], dk[16];
    const bool mine = (i >> 1) < MT;
    if (mine) {
      dw_logits(i, pk, dk);
      add_dot(i, pk, dk);
    }
    __syncthreads();
    if (mine) put_dl(i, pk, dk);
  } else {  // several tiles per wave: the row dots first, then the tiles again
#pragma unroll 1
    for (int i = wave; i < 2 * MT; i += BW) {
      float pk[16], dk[16];
      dw_logits(i, pk, dk);
      add_dot(i, pk, dk);
    }
    __syncthreads();
#pragma unroll 1
    for (int i = wave; i < 2 * MT; i += BW) {
      float pk[16], dk[16];
      dw_logits(i, pk, dk);
      put_dl(i, pk, dk);
    }
  }
  __syncthreads();

  // ---- dA^T[m][k] = sum_t w[t][m] drk[t][k] + dl[t][m] u[t][k]  -> da
  auto da_at = [&](int m, int k) -> float* {
    return q.a_first ? g.da_first + ((int64_t)q.b * H + q.h) * Dk * M + (int64_t)k * M + m
                     : g.da_states + (((int64_t)q.b * H + q.h) * N + q.n) * M * Dk + (int64_t)m * Dk + k;
  };
  for (int i = wave; i < MT * KT; i += BW) {
    const int mt = i % MT, kt = i / MT;
    f32x16 a1 = {}, a2 = {};
#pragma unroll
    for (int ts = 0; ts < LROWS / 16; ++ts) {
      const bf16x8 drk = frag_t(DRKT, 32 * kt + li, ts), u = frag_t(UT, 32 * kt + li, ts);
      a1 = mfma16(frag_t(WT, 32 * mt + li, ts), drk, a1);
      if (!given) {
        a2 = mfma16(frag_t(DLH, 32 * mt + li, ts), u, a2);
        a1 = mfma16(frag_t(DLL, 32 * mt + li, ts), u, a1);
      }
    }
    const int k = 32 * kt + li;
#pragma unroll
    for (int r = 0; r < 16; ++r) *da_at(32 * mt + acc_row(r, hh), k) = a1[r] + a2[r];
  }
  __syncthreads();  // w^T, drk^T and u^T are dead: du reuses their memory

  if (!given) {
  // ---- du[t][k] = sum_m dl[t][m] A^[k][m], dl rows gathered from dl^T.
  for (int i = wave; i < 2 * KT; i += BW) {
    const int rt = i & 1, kt = i >> 1, k = 32 * kt + li;
    const Col am = ahat_m(q, k);
    f32x16 c1 = {}, c2 = {};
    constexpr int G = 4;
#pragma unroll 1
    for (int s0 = 0; s0 < M16; s0 += G) {
      float v[G][8];
#pragma unroll
      for (int jj = 0; jj < G; ++jj) raw8<true>(am, 16 * (s0 + jj < M16 ? s0 + jj : M16 - 1) + 8 * hh, v[jj]);
#pragma unroll
      for (int jj = 0; jj < G; ++jj)
        if (s0 + jj < M16) {
          mask8(am, 16 * (s0 + jj) + 8 * hh, v[jj]);
          bf16x8 bh, bl, ah, al;
          split8(v[jj], bh, bl);
          const int m0 = 16 * (s0 + jj) + 8 * hh, t = 32 * rt + li;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            ah[e] = DLH[(m0 + e) * TP + t];
            al[e] = DLL[(m0 + e) * TP + t];
          }
          c1 = mfma16(ah, bh, c1);
          c2 = mfma16(ah, bl, c2);
          c1 = mfma16(al, bh, c1);
        }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) DU[(32 * rt + acc_row(r, hh)) * L.lde + k] = round_as<bf16_t>(c1[r] + c2[r]);
  }
  __syncthreads();

  // ---- dkey = round(dkey' + round(unit backward of du)), 16 rows per pass.
  {
    const int c = 8 * (tid & 31), r0 = tid >> 5;
    const bool on = c < Dk;
#pragma unroll
    for (int i = 0; i < LROWS / 16; ++i) {
      const int r = r0 + 16 * i, t = q.token(r);
      float x[8], du[8];
      if (on && t >= 0) bf8_to_f32(*reinterpret_cast<const uint4*>(key + q.at(p.key, t) + c), x);
      else
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = 0.f;
      const float den = den_s[r];
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        du[e] = on ? DU[r * L.lde + c + e] : 0.f;
        x[e] = x[e] / den;
        dot += x[e] * du[e];
      }
      dot = sum32(dot);
      if (!on || t < 0) continue;
      float dko[8];
      bf8_to_f32(*reinterpret_cast<const uint4*>(reinterpret_cast<const bf16_t*>(g.dkey_out.ptr) + q.at(g.dkey_out, t) + c), dko);
      const bool clamped = den <= 1e-6f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float ub = clamped ? du[e] / den : (du[e] - x[e] * dot) / den;
        dko[e] = round_as<bf16_t>(dko[e] + round_as<bf16_t>(ub));
      }
      *reinterpret_cast<uint4*>(reinterpret_cast<bf16_t*>(g.dkey.ptr) + q.at(g.dkey, t) + c) = f32_to_bf8(dko);
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
      for (int w = 0; w < BW; ++w) x += red[w][tid];
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
// Vector fragment loads need whole 16-wide contraction steps (and so 32-byte
// aligned snapshot rows).
// Rows of the activation operands are read and written as 16-byte vectors.
bool rows_aligned(const gpa_operand& o) {
  return reinterpret_cast<uintptr_t>(o.ptr) % 16 == 0 && o.sb % 8 == 0 && o.st % 8 == 0 && o.sh % 8 == 0;
}

bool level_fast(const gpa_level_problem& p) {
  return p.key_dim % 16 == 0 && p.value_dim % 16 == 0 && p.slots % 16 == 0 && rows_aligned(p.key) &&
         rows_aligned(p.value) && rows_aligned(p.write) && rows_aligned(p.key_out) && rows_aligned(p.value_out);
}

// level_bwd16: widths multiples of 32, 16-byte aligned rows, LDS within the CU.
bool level_bwd16_ok(const gpa_level_problem& p, const gpa_level_grads& g) {
  const size_t statics = 4 * LROWS * sizeof(float) + BW * 2 * sizeof(float);
  return p.key_dim % 32 == 0 && p.value_dim % 32 == 0 && p.slots % 32 == 0 && level_fast(p) &&
         rows_aligned(g.dkey_out) && rows_aligned(g.dvalue_out) && rows_aligned(g.dkey) &&
         Lds16b(p.key_dim, p.value_dim, p.slots).bytes + statics <= LDS_MAX;
}

int launch_level_fwd16(const gpa_level_problem& p, dim3 grid, hipStream_t stream) {
  const size_t lds = Lds16(p.key_dim, p.value_dim, p.slots).bytes;
  if (level_fast(p)) {
    if (int rc = level_lds(level_fwd16<true>, lds)) return rc;
    hipLaunchKernelGGL((level_fwd16<true>), grid, dim3(LNT), lds, stream, p);
  } else {
    if (int rc = level_lds(level_fwd16<false>, lds)) return rc;
    hipLaunchKernelGGL((level_fwd16<false>), grid, dim3(LNT), lds, stream, p);
  }
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
  if (!problem->key_out.ptr || !problem->value_out.ptr || (!problem->given_write && !problem->stats))
    return fail(GPA_HIP_EINVAL, "level: null output");
  const int N = (problem->offset + problem->tokens + problem->chunk - 1) / problem->chunk;
  const dim3 grid(N, problem->batch * problem->heads);
  const bool bf = problem->dtype == GPA_DTYPE_BF16, big = slab_rows(*problem, false) == 64;
  int rc = bf ? launch_level_fwd16(*problem, grid, stream)
              : (big ? launch_level_fwd<float, 64>(*problem, grid, stream)
                     : launch_level_fwd<float, 32>(*problem, grid, stream));
  if (rc) return rc;
  return check_launch("gpa_level_forward");
}

extern "C" int gpa_level_backward(const gpa_level_problem* problem, const gpa_level_grads* grads,
                                  hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_level(problem)) return rc;
  const bool given = problem->given_write != 0;
  if (!grads || !grads->dkey_out.ptr || !grads->dvalue_out.ptr ||
      (given ? !grads->dwrite_given.ptr : (!grads->dwrite.ptr || !grads->dkey.ptr || !problem->stats)) ||
      !grads->da_states ||
      !grads->db_states || !grads->deta || (problem->a_first && !grads->da_first) ||
      (problem->b_first && !grads->db_first))
    return fail(GPA_HIP_EINVAL, "level: null gradient buffer");
  const int N = (problem->offset + problem->tokens + problem->chunk - 1) / problem->chunk;
  const dim3 grid(N, problem->batch * problem->heads);
  const bool bf = problem->dtype == GPA_DTYPE_BF16, big = slab_rows(*problem, true) == 64;
  if (bf && level_bwd16_ok(*problem, *grads)) {
    const size_t lds = Lds16b(problem->key_dim, problem->value_dim, problem->slots).bytes;
    if (problem->slots <= 128) {
      if (int rc = level_lds(level_bwd16<1>, lds)) return rc;
      hipLaunchKernelGGL((level_bwd16<1>), grid, dim3(BNT), lds, stream, *problem, *grads);
    } else {
      if (int rc = level_lds(level_bwd16<2>, lds)) return rc;
      hipLaunchKernelGGL((level_bwd16<2>), grid, dim3(BNT), lds, stream, *problem, *grads);
    }
    return check_launch("gpa_level_backward");
  }
  int rc = bf ? (big ? launch_level_bwd<bf16_t, 64>(*problem, *grads, grid, stream)
                     : launch_level_bwd<bf16_t, 32>(*problem, *grads, grid, stream))
              : (big ? launch_level_bwd<float, 64>(*problem, *grads, grid, stream)
                     : launch_level_bwd<float, 32>(*problem, *grads, grid, stream));
  if (rc) return rc;
  return check_launch("gpa_level_backward");
}
