// Route reader of one target level: forward, backward and weight gradients of
// the default read of the reference's _bridge (src/gpa/attention.py:225-262,
// legacy branch :236-240; the closed form of packed.py:16-35).
//
// A workgroup owns 32 token rows of one head.  Row phases (8 threads per
// row) do the per-row softmax and normalisation work; the four products per
// row tile (r0 U, gelu(h1) D, r1 W_rs, q W_qs in the forward; their
// transposes in the backward) run as 32x32 output tiles on MFMA, A rows from
// LDS and B rows from the padded weight matrices (L2-resident, shared by all
// row tiles of a head).  Every product rounds its operands and result to the
// activation type and accumulates in float32, as the reference's typed
// einsums do; the gradients round where the reference's bf16 tensors do.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "mfma_tiles.h"

namespace gpa {
namespace {

constexpr int RR = GPA_ROUTE_ROWS;  // token rows per workgroup
constexpr int RW = 4;               // waves per workgroup
constexpr int RNT = 64 * RW;
constexpr int RMAX = GPA_ROUTE_MAX_WIDTH;
constexpr int RPER = RMAX / 8;      // columns per thread in a row phase (8 threads per row)
constexpr int RTMAX = RMAX / 32 / RW;  // M-column tiles per wave (at most)

__host__ __device__ constexpr int pad16(int x) { return (x + 15) & ~15; }
__host__ __device__ constexpr int pad32(int x) { return (x + 31) & ~31; }

template <typename E> struct Wt;
template <> struct Wt<float> { using type = float; };
template <> struct Wt<bf16_t> { using type = bf16_t; };

// acc += A[32][K] B, A rows in LDS (already in the activation type's values,
// zero beyond K up to k16), B given as rows bt[n0 + c][0..k16) (zero padded).
// The B fragments of up to 8 contraction steps are loaded before their MFMAs,
// so that their latency overlaps.
__device__ __forceinline__ void tile_gemm(f32x16& acc, const float* a, int lda, const bf16_t* bt, int ldb,
                                          int k16, int n0, int lane) {
  const float* ar = a + (lane & 31) * lda + 8 * (lane >> 5);
  const bf16_t* br = bt + (int64_t)(n0 + (lane & 31)) * ldb + 8 * (lane >> 5);
  for (int k0 = 0; k0 < k16; k0 += 8 * 16) {
    bf16x8 bv[8];
#pragma unroll
    for (int s = 0; s < 8; ++s)
      if (k0 + 16 * s < k16) bv[s] = *reinterpret_cast<const bf16x8*>(br + k0 + 16 * s);
#pragma unroll
    for (int s = 0; s < 8; ++s)
      if (k0 + 16 * s < k16)
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pack8(ar + k0 + 16 * s), bv[s], acc, 0, 0, 0);
  }
}
__device__ __forceinline__ void tile_gemm(f32x16& acc, const float* a, int lda, const float* bt, int ldb, int k16,
                                          int n0, int lane) {
  const float* ar = a + (lane & 31) * lda + 4 * (lane >> 5);
  const float* br = bt + (int64_t)(n0 + (lane & 31)) * ldb + 4 * (lane >> 5);
  for (int k0 = 0; k0 < k16; k0 += 8 * 8) {
    f32x4 bv[8];
#pragma unroll
    for (int s = 0; s < 8; ++s)
      if (k0 + 8 * s < k16) bv[s] = *reinterpret_cast<const f32x4*>(br + k0 + 8 * s);
#pragma unroll
    for (int s = 0; s < 8; ++s)
      if (k0 + 8 * s < k16) mma8(acc, *reinterpret_cast<const f32x4*>(ar + k0 + 8 * s), bv[s]);
  }
}

__device__ __forceinline__ float sum8(float x) {
  x += __shfl_xor(x, 1);
  x += __shfl_xor(x, 2);
  return x + __shfl_xor(x, 4);
}
__device__ __forceinline__ float max8(float x) {
  x = fmaxf(x, __shfl_xor(x, 1));
  x = fmaxf(x, __shfl_xor(x, 2));
  return fmaxf(x, __shfl_xor(x, 4));
}

__device__ __forceinline__ float gelu(float x) { return .5f * x * (1.f + erff(x * 0.70710678118654752f)); }
__device__ __forceinline__ float gelu_grad(float x) {
  return .5f * (1.f + erff(x * 0.70710678118654752f)) + x * 0.39894228040143268f * __expf(-.5f * x * x);
}

// Workgroups go to the 8 XCDs round robin (id % 8).  xcd_logical renumbers
// them so that each XCD runs a contiguous range of logical ids, and
// workgroups that read the same data (one head's weights; the tiles of one
// weight-gradient product, head and span) share that XCD's L2.
__device__ __forceinline__ int xcd_logical(int id, int n) {
  const int q = n / 8, r = n % 8, x = id % 8, local = id / 8;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + local;
}
// Row tile and head of a route workgroup (grid: row tiles x heads).
struct RouteTile {
  int tile, h;
};
__device__ __forceinline__ RouteTile route_tile() {
  const int nt = gridDim.x, id = xcd_logical(blockIdx.x + nt * blockIdx.y, nt * gridDim.y);
  return RouteTile{id % nt, id / nt};
}

// Offsets of a workgroup's rows r = b*T + t: the (b, t) split of each of its
// RR rows is computed once (rows past the end repeat the last one).
struct Rows {
  int row0;
  const int *rb, *rt;
  __device__ __forceinline__ int64_t at(const gpa_operand& o, int r, int h) const {
    const int i = r - row0;
    return (int64_t)rb[i] * o.sb + (int64_t)rt[i] * o.st + (int64_t)h * o.sh;
  }
};

__device__ __forceinline__ Rows make_rows(int* rb, int* rt, int row0, int R, int T) {
  if (threadIdx.x < RR) {
    const int r = row0 + threadIdx.x < R ? row0 + threadIdx.x : R - 1;
    rb[threadIdx.x] = r / T;
    rt[threadIdx.x] = r % T;
  }
  __syncthreads();
  return Rows{row0, rb, rt};
}

// Relation read and softmax of one row (8 threads, columns part + 8 i):
// returns base' = base + gain tanh z in v[], and fills z[] / inc[] when asked.
template <typename E>
__device__ __forceinline__ void row_base(const gpa_route_problem& p, const Rows& rows, int r, int h, int part,
                                         float (&v)[RPER], float (&z)[RPER], float& inv_sig) {
  const int M = p.slots;
  const float* base = reinterpret_cast<const float*>(p.base.ptr) + rows.at(p.base, r, h);
#pragma unroll
  for (int i = 0; i < RPER; ++i) {
    const int m = part + 8 * i;
    v[i] = m < M ? base[m] : 0.f;
    z[i] = 0.f;
  }
  inv_sig = 0.f;
  if (p.incoming == 0) return;
  for (int e = 0; e < p.incoming; ++e) {
    const float w = p.edge_weight[e * p.heads + h];
    const E* msg = reinterpret_cast<const E*>(p.msg[e].ptr) + rows.at(p.msg[e], r, h);
#pragma unroll
    for (int i = 0; i < RPER; ++i) {
      const int m = part + 8 * i;
      if (m < M) z[i] += w * to_f32(msg[m]);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < RPER; ++i) s += z[i];
  const float mean = sum8(s) / M;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < RPER; ++i) {
    const int m = part + 8 * i;
    z[i] = m < M ? z[i] - mean : 0.f;
    q += z[i] * z[i];
  }
  const float sig = sqrtf(sum8(q) / M + 1e-5f);
  inv_sig = 1.f / sig;
  const float gain = p.gain[h];
#pragma unroll
  for (int i = 0; i < RPER; ++i) {
    z[i] = z[i] / sig;
    v[i] += gain * tanhf(z[i]);
  }
}

template <typename E>
__device__ __forceinline__ void row_softmax(int M, int part, const float (&v)[RPER], float (&pr)[RPER]) {
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < RPER; ++i)
    if (part + 8 * i < M) mx = fmaxf(mx, v[i]);
  mx = max8(mx);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < RPER; ++i) {
    pr[i] = part + 8 * i < M ? __expf(v[i] - mx) : 0.f;
    s += pr[i];
  }
  s = sum8(s);
#pragma unroll
  for (int i = 0; i < RPER; ++i) pr[i] /= s;
}

// VEC (bf16 activations, widths multiples of 8, 16-byte aligned rows): the
// row phases run with 32 lanes per row, 8 columns each, every 16-byte load of
// a thread issued before its first use.
constexpr int VPASS = RR / (RNT / 32);  // row passes of 8 rows

__device__ __forceinline__ float vsum32(float x) {
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) x += __shfl_xor(x, m, 32);
  return x;
}
__device__ __forceinline__ float vmax32(float x) {
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m, 32));
  return x;
}
__device__ __forceinline__ void unpack_bf8(const uint4& u, float (&x)[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = __uint_as_float(w[i] << 16);
    x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ uint4 pack_bf8(const float (&x)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = (uint32_t)f32_to_bf16(x[2 * i]).bits | ((uint32_t)f32_to_bf16(x[2 * i + 1]).bits << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// r0 = softmax(base + gain tanh z) of a workgroup's RR rows, rounded to E,
// with 32 lanes per row (8 columns each) and 8 rows per pass (VEC rows):
// written to the saved rows sr0 and, when A is given, to the LDS tile
// A [RR][lda] (zero beyond M, up to kM).
template <typename E>
__device__ __forceinline__ void rows_r0_vec(const gpa_route_problem& p, const Rows& rows, int row0, int h,
                                            E* sr0, float* A, int lda, int kM) {
  const int M = p.slots, R = p.batch * p.tokens, tid = threadIdx.x;
  const int c = 8 * (tid & 31), rsub = tid >> 5;
  const bool on = c < M;
  float bv[VPASS][8];
  uint4 mv[VPASS][GPA_ROUTE_MAX_INCOMING];
#pragma unroll
  for (int i = 0; i < VPASS; ++i) {
    const int r = row0 + rsub + 8 * i, rr = r < R ? r : R - 1;
    if (on) {
      const float* bp = reinterpret_cast<const float*>(p.base.ptr) + rows.at(p.base, rr, h) + c;
      const f32x4 x0 = *reinterpret_cast<const f32x4*>(bp), x1 = *reinterpret_cast<const f32x4*>(bp + 4);
      bv[i][0] = x0.x; bv[i][1] = x0.y; bv[i][2] = x0.z; bv[i][3] = x0.w;
      bv[i][4] = x1.x; bv[i][5] = x1.y; bv[i][6] = x1.z; bv[i][7] = x1.w;
#pragma unroll
      for (int e = 0; e < GPA_ROUTE_MAX_INCOMING; ++e)
        if (e < p.incoming)
          mv[i][e] = *reinterpret_cast<const uint4*>(reinterpret_cast<const bf16_t*>(p.msg[e].ptr) +
                                                     rows.at(p.msg[e], rr, h) + c);
    }
  }
  const float gain = p.gain[h];
  // edge weights read once (a load inside the row loop would wait behind the stores)
  float ew[GPA_ROUTE_MAX_INCOMING];
#pragma unroll
  for (int e = 0; e < GPA_ROUTE_MAX_INCOMING; ++e) ew[e] = e < p.incoming ? p.edge_weight[e * p.heads + h] : 0.f;
#pragma unroll
  for (int i = 0; i < VPASS; ++i) {
    const int row = rsub + 8 * i, r = row0 + row;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = on ? bv[i][e] : 0.f;
    if (p.incoming > 0) {
      float z[8] = {};
#pragma unroll
      for (int e = 0; e < GPA_ROUTE_MAX_INCOMING; ++e)
        if (e < p.incoming && on) {
          const float w = ew[e];
          float x[8];
          unpack_bf8(mv[i][e], x);
#pragma unroll
          for (int j = 0; j < 8; ++j) z[j] += w * x[j];
        }
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) s += z[j];
      const float mean = vsum32(s) / M;
      float qq = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        z[j] = on ? z[j] - mean : 0.f;
        qq += z[j] * z[j];
      }
      const float sig = sqrtf(vsum32(qq) / M + 1e-5f);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] += gain * tanhf(z[j] / sig);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) mx = on ? fmaxf(mx, v[j]) : mx;
    mx = vmax32(mx);
    float sm = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[j] = on ? __expf(v[j] - mx) : 0.f;
      sm += v[j];
    }
    sm = vsum32(sm);
    const bool valid = r < R;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (valid && on) ? round_as<E>(v[j] / sm) : 0.f;
    if (A && c < kM) {
      *reinterpret_cast<f32x4*>(&A[row * lda + c]) = f32x4{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<f32x4*>(&A[row * lda + c + 4]) = f32x4{v[4], v[5], v[6], v[7]};
    }
    if (valid && on) *reinterpret_cast<uint4*>(sr0 + (int64_t)r * M + c) = pack_bf8(v);
  }
}

// Softmax and relation-read backward of a workgroup's RR rows (VEC rows: 32
// lanes per row, 8 columns each, 8 rows per pass) from d r0 (d0v[pass][j],
// the lane's columns of row rsub + 8 pass): writes d base and the message
// gradients, and adds the lane's shares of d gain and d w_e.
template <typename E>
__device__ __forceinline__ void rows_bwd_vec(const gpa_route_problem& p, const gpa_route_grads& g, const Rows& rows,
                                             int row0, int h, const float (&d0v)[VPASS][8], float& part_gain,
                                             float (&part_w)[GPA_ROUTE_MAX_INCOMING]) {
  const int M = p.slots, R = p.batch * p.tokens, H = p.heads, NI = p.incoming, tid = threadIdx.x;
  const int c = 8 * (tid & 31), rsub = tid >> 5;
  const bool on = c < M;
  float bv[VPASS][8];
  uint4 mv[VPASS][GPA_ROUTE_MAX_INCOMING];
#pragma unroll
  for (int i = 0; i < VPASS; ++i) {
    const int r = row0 + rsub + 8 * i, rr = r < R ? r : R - 1;
    if (on) {
      const float* bp = reinterpret_cast<const float*>(p.base.ptr) + rows.at(p.base, rr, h) + c;
      const f32x4 x0 = *reinterpret_cast<const f32x4*>(bp), x1 = *reinterpret_cast<const f32x4*>(bp + 4);
      bv[i][0] = x0.x; bv[i][1] = x0.y; bv[i][2] = x0.z; bv[i][3] = x0.w;
      bv[i][4] = x1.x; bv[i][5] = x1.y; bv[i][6] = x1.z; bv[i][7] = x1.w;
#pragma unroll
      for (int e = 0; e < GPA_ROUTE_MAX_INCOMING; ++e)
        if (e < NI)
          mv[i][e] = *reinterpret_cast<const uint4*>(reinterpret_cast<const bf16_t*>(p.msg[e].ptr) +
                                                     rows.at(p.msg[e], rr, h) + c);
    }
  }
  const float gain = p.gain[h];
  float ew[GPA_ROUTE_MAX_INCOMING];  // read once, as in the forward
#pragma unroll
  for (int e = 0; e < GPA_ROUTE_MAX_INCOMING; ++e) ew[e] = e < NI ? p.edge_weight[e * H + h] : 0.f;
#pragma unroll
  for (int i = 0; i < VPASS; ++i) {
    const int row = rsub + 8 * i, r = row0 + row;
    const bool valid = r < R;
    float v[8], z[8] = {}, thz[8] = {}, msgf[GPA_ROUTE_MAX_INCOMING][8], inv = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = on ? bv[i][e] : 0.f;
    if (NI > 0) {
#pragma unroll
      for (int e = 0; e < GPA_ROUTE_MAX_INCOMING; ++e)
        if (e < NI && on) {
          const float w = ew[e];
          unpack_bf8(mv[i][e], msgf[e]);
#pragma unroll
          for (int j = 0; j < 8; ++j) z[j] += w * msgf[e][j];
        }
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) s += z[j];
      const float mean = vsum32(s) / M;
      float qq = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        z[j] = on ? z[j] - mean : 0.f;
        qq += z[j] * z[j];
      }
      const float sig = sqrtf(vsum32(qq) / M + 1e-5f);
      inv = 1.f / sig;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        z[j] = z[j] / sig;
        thz[j] = tanhf(z[j]);
        v[j] += gain * thz[j];
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) mx = on ? fmaxf(mx, v[j]) : mx;
    mx = vmax32(mx);
    float pr[8], sm = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pr[j] = on ? __expf(v[j] - mx) : 0.f;
      sm += pr[j];
    }
    sm = vsum32(sm);
    float d0[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) d0[j] = on ? d0v[i][j] : 0.f;
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pr[j] /= sm;
      s += pr[j] * d0[j];
    }
    s = vsum32(s);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = on ? pr[j] * (d0[j] - s) : 0.f;  // d base'
    if (valid && on) {
      float* db = reinterpret_cast<float*>(g.dbase.ptr) + rows.at(g.dbase, r, h) + c;
      *reinterpret_cast<f32x4*>(db) = f32x4{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<f32x4*>(db + 4) = f32x4{v[4], v[5], v[6], v[7]};
    }
    if (NI > 0) {
      float dz[8], szz = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float th = thz[j];
        if (valid && on) part_gain += v[j] * th;
        dz[j] = on ? gain * v[j] * (1.f - th * th) : 0.f;
        szz += dz[j] * z[j];
      }
      const float mzz = vsum32(szz) / M;
      float sc = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        dz[j] = on ? (dz[j] - z[j] * mzz) * inv : 0.f;  // d centred
        sc += dz[j];
      }
      const float mc = vsum32(sc) / M;
#pragma unroll
      for (int j = 0; j < 8; ++j) dz[j] -= mc;  // d incoming
#pragma unroll
      for (int e = 0; e < GPA_ROUTE_MAX_INCOMING; ++e)
        if (e < NI && on) {
          const float w = ew[e];
          float sw = 0.f, dm[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            sw += dz[j] * msgf[e][j];
            dm[j] = round_as<E>(w * dz[j]);
          }
          if (valid) {
            part_w[e] += sw;
            *reinterpret_cast<uint4*>(reinterpret_cast<bf16_t*>(g.dmsg[e].ptr) + rows.at(g.dmsg[e], r, h) + c) =
                pack_bf8(dm);
          }
        }
    }
  }
}

// The forward of RR rows (row0 ..) of head h of one problem.
// NW waves: the row phases and the q staging run on the first RNT threads,
// the product tiles are spread over all NW waves (the packed one-token read
// uses 8, so that the 32 rows of a wide level walk half as many tiles per wave).
template <typename E, bool VEC, int NW = RW>
__device__ __forceinline__ void route_fwd_run(const gpa_route_problem& p, int h, int row0) {
  using W = typename Wt<E>::type;
  HIP_DYNAMIC_SHARED(float, lds)
  const int M = p.slots, Dk = p.key_dim, R = p.batch * p.tokens;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kM = pad16(M), k2M = pad16(2 * M), kD = pad16(Dk);
  const int lda = kM + 4, ldh = (k2M > kD ? k2M : kD) + 4;
  float* A = lds;             // r0, then r1        [RR][lda]
  float* Hs = lds + RR * lda; // gelu(h1), then q   [RR][ldh]
  __shared__ int row_b[RR], row_t[RR];
  const Rows rows = make_rows(row_b, row_t, row0, R, p.tokens);
  E* sr0 = reinterpret_cast<E*>(p.r0) + (int64_t)h * R * M;
  E* sh1 = reinterpret_cast<E*>(p.h1) + (int64_t)h * R * 2 * M;
  E* shd = reinterpret_cast<E*>(p.hd) + (int64_t)h * R * M;

  // ---- r0 = softmax(base + gain tanh z)
  if (NW > RW && tid >= RNT) {
    // the row phase runs on the first RNT threads
  } else if constexpr (VEC) {
    rows_r0_vec<E>(p, rows, row0, h, sr0, A, lda, kM);
  } else {
    const int row = tid >> 3, part = tid & 7, r = row0 + row;
    const bool valid = r < R;
    float v[RPER], z[RPER], pr[RPER], inv;
    row_base<E>(p, rows, valid ? r : R - 1, h, part, v, z, inv);
    row_softmax<E>(M, part, v, pr);
#pragma unroll
    for (int i = 0; i < RPER; ++i) {
      const int m = part + 8 * i;
      if (m < kM) {
        const float x = (valid && m < M) ? round_as<E>(pr[i]) : 0.f;
        A[row * lda + m] = x;
        if (valid && m < M) sr0[(int64_t)r * M + m] = from_f32<E>(x);
      }
    }
  }
  __syncthreads();

  // ---- h1 = r0 U, gelu(h1) -> Hs
  {
    const W* ut = reinterpret_cast<const W*>(p.up_t) + (int64_t)h * pad32(2 * M) * kM;
    for (int t = wave; t < pad32(2 * M) / 32; t += NW) {
      f32x16 acc = {};
      tile_gemm(acc, A, lda, ut, kM, kM, 32 * t, lane);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = acc_row(i, lane >> 5), col = 32 * t + (lane & 31), r = row0 + row;
        if (col < 2 * M) {
          const float h1 = round_as<E>(acc[i]);
          if (r < R) sh1[(int64_t)r * 2 * M + col] = from_f32<E>(h1);
          Hs[row * ldh + col] = round_as<E>(gelu(h1));
        } else if (col < k2M) {
          Hs[row * ldh + col] = 0.f;
        }
      }
    }
  }
  __syncthreads();

  // ---- hd = gelu(h1) D, r1 = r0 + mlp_gain hd -> A and the route output
  {
    const W* dt = reinterpret_cast<const W*>(p.down_t) + (int64_t)h * pad32(M) * k2M;
    const float g = p.mlp_gain[h];
    E* route = reinterpret_cast<E*>(p.route.ptr);
    for (int t = wave; t < pad32(M) / 32; t += NW) {
      f32x16 acc = {};
      tile_gemm(acc, Hs, ldh, dt, k2M, k2M, 32 * t, lane);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = acc_row(i, lane >> 5), col = 32 * t + (lane & 31), r = row0 + row;
        if (col < M) {
          const float hd = round_as<E>(acc[i]);
          const float r1 = round_as<E>(A[row * lda + col] + g * hd);
          A[row * lda + col] = r1;
          if (r < R) {
            shd[(int64_t)r * M + col] = from_f32<E>(hd);
            if (!p.rsa) route[rows.at(p.route, r, h) + col] = from_f32<E>(r1);
          }
        }
      }
    }
  }
  __syncthreads();

  // ---- rsa_update: r1 <- round(r1 / clamp(sum |r1|, .25, 4)) in A and the route output
  if (p.rsa) {
    if (!(NW > RW && tid >= RNT)) {
      const int row = tid >> 3, part = tid & 7, r = row0 + row;
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < RPER; ++i)
        if (part + 8 * i < M) s += fabsf(A[row * lda + part + 8 * i]);
      const float l = fminf(fmaxf(sum8(s), .25f), 4.f);
      E* route = reinterpret_cast<E*>(p.route.ptr);
#pragma unroll
      for (int i = 0; i < RPER; ++i) {
        const int m = part + 8 * i;
        if (m < M) {
          const float x = round_as<E>(A[row * lda + m] / l);
          A[row * lda + m] = x;
          if (r < R) route[rows.at(p.route, r, h) + m] = from_f32<E>(x);
        }
      }
    }
    __syncthreads();
  }

  // ---- q -> Hs
  if (NW > RW && tid >= RNT) {
    // the q staging runs on the first RNT threads
  } else if constexpr (VEC) {
    const int c = 8 * (tid & 31), rsub = tid >> 5;
    uint4 qv[VPASS];
#pragma unroll
    for (int i = 0; i < VPASS; ++i) {
      const int r = row0 + rsub + 8 * i;
      qv[i] = (c < Dk && r < R) ? *reinterpret_cast<const uint4*>(reinterpret_cast<const bf16_t*>(p.q.ptr) +
                                                                   rows.at(p.q, r, h) + c)
                                : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < VPASS; ++i) {
      const int row = rsub + 8 * i;
      float x[8];
      unpack_bf8(qv[i], x);
      if (c < kD) {
        *reinterpret_cast<f32x4*>(&Hs[row * ldh + c]) = f32x4{x[0], x[1], x[2], x[3]};
        *reinterpret_cast<f32x4*>(&Hs[row * ldh + c + 4]) = f32x4{x[4], x[5], x[6], x[7]};
      }
    }
  } else {
    const int row = tid >> 3, part = tid & 7, r = row0 + row;
    const bool valid = r < R;
    const E* q = reinterpret_cast<const E*>(p.q.ptr) + rows.at(p.q, valid ? r : R - 1, h);
#pragma unroll
    for (int i = 0; i < RPER; ++i) {
      const int d = part + 8 * i;
      if (d < kD) Hs[row * ldh + d] = (valid && d < Dk) ? to_f32(q[d]) : 0.f;
    }
  }
  __syncthreads();

  // ---- qo = r1 W_rs + query_scale (q W_qs)
  {
    const W* rt = reinterpret_cast<const W*>(p.rs_t) + (int64_t)h * pad32(M) * kM;
    const W* qt = reinterpret_cast<const W*>(p.qs_t) + (int64_t)h * pad32(M) * kD;
    E* qo = reinterpret_cast<E*>(p.qo.ptr);
    for (int t = wave; t < pad32(M) / 32; t += NW) {
      f32x16 a3 = {}, a4 = {};
      tile_gemm(a3, A, lda, rt, kM, kM, 32 * t, lane);
      tile_gemm(a4, Hs, ldh, qt, kD, kD, 32 * t, lane);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = acc_row(i, lane >> 5), col = 32 * t + (lane & 31), r = row0 + row;
        if (col < M && r < R) {
          const float dir = round_as<E>(p.query_scale * round_as<E>(a4[i]));
          if (p.balanced) {  // both halves saved; route_mix_fwd forms qo from their unit rows
            reinterpret_cast<E*>(p.qr)[((int64_t)h * R + r) * M + col] = from_f32<E>(round_as<E>(a3[i]));
            reinterpret_cast<E*>(p.qdir)[((int64_t)h * R + r) * M + col] = from_f32<E>(dir);
          } else {
            qo[rows.at(p.qo, r, h) + col] = from_f32<E>(round_as<E>(round_as<E>(a3[i]) + dir));
          }
        }
      }
    }
  }
}

template <typename E, bool VEC>
__global__ __launch_bounds__(RNT) void route_fwd(gpa_route_problem p) {
  const RouteTile rtile = route_tile();
  route_fwd_run<E, VEC>(p, rtile.h, rtile.tile * RR);
}

// Several problems (the target levels of one call) in one launch: workgroups
// wg0[i] .. wg0[i+1]-1 run problem i, head-major over its row tiles.  The
// problem is read through the kernel-argument pointer with a uniform offset
// (indexing the by-value argument would copy it to scratch).
struct RoutePack {
  int n;
  int wg0[GPA_ROUTE_MAX_PACK], tiles[GPA_ROUTE_MAX_PACK];
  gpa_route_problem p[GPA_ROUTE_MAX_PACK];
};

typedef const __attribute__((address_space(4))) RoutePack* RoutePackPtr;

// The pack entry of this workgroup, copied word by word from the argument segment.
__device__ __forceinline__ int route_pack_entry(RoutePackPtr kp, gpa_route_problem& p) {
  int pi = 0;
#pragma unroll 1
  for (int i = 1; i < kp->n; ++i)
    if ((int)blockIdx.x >= kp->wg0[i]) pi = i;
  const __attribute__((address_space(4))) uint32_t* src =
      (const __attribute__((address_space(4))) uint32_t*)&kp->p[pi];
  uint32_t* dst = reinterpret_cast<uint32_t*>(&p);
#pragma unroll
  for (int i = 0; i < (int)(sizeof(gpa_route_problem) / 4); ++i) dst[i] = src[i];
  return pi;
}

// bf16 with 16-byte rows (the one-token decode path), 8 waves per workgroup.
constexpr int RPACK_W = 8;
__global__ __launch_bounds__(64 * RPACK_W) void route_fwd_pack(RoutePack pk) {
  const RoutePackPtr kp = (RoutePackPtr)__builtin_amdgcn_kernarg_segment_ptr();
  gpa_route_problem p;
  const int pi = route_pack_entry(kp, p);
  const int local = (int)blockIdx.x - kp->wg0[pi], nt = kp->tiles[pi];
  route_fwd_run<bf16_t, true, RPACK_W>(p, local / nt, (local % nt) * RR);
}

// ---------------------------------------------------------------- rsa_update and balanced_bridge rows
// The two reference flags that act on whole rows between the products (sums
// over the M slots), as row kernels: 8 threads per row, the RR rows of one
// head per workgroup (grid: row tiles x heads).  Products and sums whose
// rounding the reference fixes are written with mul_rn / add_rn (no FMA
// contraction).

struct RowCtx {
  int M, R, h, tile, row, part, r, rc;
};
__device__ __forceinline__ RowCtx row_ctx(const gpa_route_problem& p) {
  const RouteTile t = route_tile();
  const int R = p.batch * p.tokens, row = threadIdx.x >> 3, r = t.tile * RR + row;
  return RowCtx{p.slots, R, t.h, t.tile, row, (int)threadIdx.x & 7, r, r < R ? r : R - 1};
}

// rsa_update forward (attention.py:251-253), in place on the route rows:
// r1 <- round(r1 / clamp(sum |r1|, .25, 4)).  (The one-kernel reader does the
// same in its LDS tile.)
template <typename E>
__global__ __launch_bounds__(RNT) void route_rsa_fwd(gpa_route_problem p) {
  const RowCtx c = row_ctx(p);
  __shared__ int row_b[RR], row_t[RR];
  const Rows rows = make_rows(row_b, row_t, c.tile * RR, c.R, p.tokens);
  E* route = reinterpret_cast<E*>(p.route.ptr) + rows.at(p.route, c.rc, c.h);
  float x[RPER], s = 0.f;
#pragma unroll
  for (int i = 0; i < RPER; ++i) {
    const int m = c.part + 8 * i;
    x[i] = m < c.M ? to_f32(route[m]) : 0.f;
    s += fabsf(x[i]);
  }
  const float l = fminf(fmaxf(sum8(s), .25f), 4.f);
  if (c.r < c.R) {
#pragma unroll
    for (int i = 0; i < RPER; ++i)
      if (c.part + 8 * i < c.M) route[c.part + 8 * i] = from_f32<E>(round_as<E>(x[i] / l));
  }
}

// One row's |x| = sqrt(sum x^2) over the thread's columns and its 7 partners.
__device__ __forceinline__ float row_norm(const float (&x)[RPER]) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < RPER; ++i) s += x[i] * x[i];
  return sqrtf(sum8(s));
}

// balanced_bridge forward (attention.py:256-259):
// qo = round(mix unit(qr) + (1 - mix) unit(qdir)), unit(x) = round(x / max(|x|, 1e-6)).
template <typename E>
__global__ __launch_bounds__(RNT) void route_mix_fwd(gpa_route_problem p) {
  const RowCtx c = row_ctx(p);
  __shared__ int row_b[RR], row_t[RR];
  const Rows rows = make_rows(row_b, row_t, c.tile * RR, c.R, p.tokens);
  const int64_t o = ((int64_t)c.h * c.R + c.rc) * c.M;
  const E* qr = reinterpret_cast<const E*>(p.qr) + o;
  const E* qd = reinterpret_cast<const E*>(p.qdir) + o;
  float a[RPER], b[RPER];
#pragma unroll
  for (int i = 0; i < RPER; ++i) {
    const int m = c.part + 8 * i;
    a[i] = m < c.M ? to_f32(qr[m]) : 0.f;
    b[i] = m < c.M ? to_f32(qd[m]) : 0.f;
  }
  const float na = fmaxf(row_norm(a), 1e-6f), nb = fmaxf(row_norm(b), 1e-6f);
  const float mix = p.mix[c.h], omix = 1.f - mix;
  E* qo = reinterpret_cast<E*>(p.qo.ptr) + rows.at(p.qo, c.rc, c.h);
  if (c.r < c.R) {
#pragma unroll
    for (int i = 0; i < RPER; ++i) {
      const int m = c.part + 8 * i;
      if (m < c.M) {
        const float ua = round_as<E>(a[i] / na), ub = round_as<E>(b[i] / nb);
        qo[m] = from_f32<E>(round_as<E>(add_rn(mul_rn(mix, ua), mul_rn(omix, ub))));
      }
    }
  }
}

// Gradient of unit(x) = x / c, c = max(|x|, eps), n = |x| (F.normalize's
// autograd): dx = du / c + [n >= eps] (-sum(du x) / c^2) x / n.
__device__ __forceinline__ void unit_bwd(const float (&x)[RPER], const float (&du)[RPER], float n, float (&dx)[RPER]) {
  const float cl = fmaxf(n, 1e-6f);
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < RPER; ++i) t += du[i] * x[i];
  t = sum8(t);
  const float dn = n >= 1e-6f ? -t / (cl * cl) : 0.f;
#pragma unroll
  for (int i = 0; i < RPER; ++i) dx[i] = du[i] / cl + (n > 0.f ? dn * x[i] / n : 0.f);
}

// balanced_bridge backward, before the products: from dqo, the gradients of
// qr and qdir (rounded to E) and the block's sum of dqo . (unit(qr) - unit(qdir))
// (d mix; the reference's d mix - d (1 - mix)).
template <typename E>
__global__ __launch_bounds__(RNT) void route_mix_bwd(gpa_route_problem p, gpa_route_grads g) {
  const RowCtx c = row_ctx(p);
  __shared__ int row_b[RR], row_t[RR];
  __shared__ float red[RW];
  const Rows rows = make_rows(row_b, row_t, c.tile * RR, c.R, p.tokens);
  const int64_t o = ((int64_t)c.h * c.R + c.rc) * c.M;
  const E* qr = reinterpret_cast<const E*>(p.qr) + o;
  const E* qd = reinterpret_cast<const E*>(p.qdir) + o;
  const E* dqo = reinterpret_cast<const E*>(g.dqo.ptr) + rows.at(g.dqo, c.rc, c.h);
  float a[RPER], b[RPER], d[RPER];
#pragma unroll
  for (int i = 0; i < RPER; ++i) {
    const int m = c.part + 8 * i;
    a[i] = m < c.M ? to_f32(qr[m]) : 0.f;
    b[i] = m < c.M ? to_f32(qd[m]) : 0.f;
    d[i] = m < c.M ? to_f32(dqo[m]) : 0.f;
  }
  const float na = row_norm(a), nb = row_norm(b);
  const float ca = fmaxf(na, 1e-6f), cb = fmaxf(nb, 1e-6f);
  const float mix = p.mix[c.h], omix = 1.f - mix;
  float dua[RPER], dub[RPER], part = 0.f;
#pragma unroll
  for (int i = 0; i < RPER; ++i) {
    const bool on = c.part + 8 * i < c.M;
    const float ua = on ? round_as<E>(a[i] / ca) : 0.f, ub = on ? round_as<E>(b[i] / cb) : 0.f;
    part += d[i] * ua - d[i] * ub;
    dua[i] = on ? round_as<E>(mul_rn(d[i], mix)) : 0.f;
    dub[i] = on ? round_as<E>(mul_rn(d[i], omix)) : 0.f;
  }
  float dxa[RPER], dxb[RPER];
  unit_bwd(a, dua, na, dxa);
  unit_bwd(b, dub, nb, dxb);
  if (c.r < c.R) {
    E* gq = reinterpret_cast<E*>(g.dqr.ptr) + rows.at(g.dqr, c.r, c.h);
    E* gd = reinterpret_cast<E*>(g.ddir.ptr) + rows.at(g.ddir, c.r, c.h);
#pragma unroll
    for (int i = 0; i < RPER; ++i) {
      const int m = c.part + 8 * i;
      if (m < c.M) {
        gq[m] = from_f32<E>(round_as<E>(dxa[i]));
        gd[m] = from_f32<E>(round_as<E>(dxb[i]));
      }
    }
  } else {
    part = 0.f;
  }
  for (int k = 32; k >= 1; k >>= 1) part += __shfl_xor(part, k);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = part;
  __syncthreads();
  if (threadIdx.x == 0) g.mix_partials[(int64_t)c.tile * p.heads + c.h] = red[0] + red[1] + red[2] + red[3];
}

// rsa_update backward of one row, given d r1' (the gradient of the rescaled
// row) and r1: d r1 = round(d r1' / l + [.25 <= s <= 4] (-sum(d r1' r1) / l^2) sign(r1)),
// s = sum |r1|, l = clamp(s, .25, 4).
template <typename E>
__device__ __forceinline__ void rsa_bwd_row(const float (&r1)[RPER], const float (&d)[RPER], int M, int part,
                                            float (&out)[RPER]) {
  float s = 0.f, t = 0.f;
#pragma unroll
  for (int i = 0; i < RPER; ++i) {
    s += fabsf(r1[i]);
    t += d[i] * r1[i];
  }
  s = sum8(s);
  t = sum8(t);
  const float l = fminf(fmaxf(s, .25f), 4.f);
  const float dl = (s >= .25f && s <= 4.f) ? -t / (l * l) : 0.f;
#pragma unroll
  for (int i = 0; i < RPER; ++i) {
    const float sg = r1[i] > 0.f ? 1.f : (r1[i] < 0.f ? -1.f : 0.f);
    out[i] = part + 8 * i < M ? round_as<E>(d[i] / l + dl * sg) : 0.f;
  }
}

// rsa_update backward of the tiled path: d r1' (float32 d base rows, written
// by the d r1 product) -> d r1 in place, d hd = round(mlp_gain d r1), and the
// block's sum of d r1 . hd (partial slot 0, d mlp_gain).  r1 is recomputed
// from the saved r0 and hd rows.
template <typename E>
__global__ __launch_bounds__(RNT) void route_rsa_bwd(gpa_route_problem p, gpa_route_grads g) {
  const RowCtx c = row_ctx(p);
  __shared__ int row_b[RR], row_t[RR];
  __shared__ float red[RW];
  const Rows rows = make_rows(row_b, row_t, c.tile * RR, c.R, p.tokens);
  const int64_t o = ((int64_t)c.h * c.R + c.rc) * c.M;
  const E* r0 = reinterpret_cast<const E*>(p.r0) + o;
  const E* hd = reinterpret_cast<const E*>(p.hd) + o;
  float* dr = reinterpret_cast<float*>(g.dbase.ptr) + rows.at(g.dbase, c.rc, c.h);
  const float gm = p.mlp_gain[c.h];
  float r1[RPER], hv[RPER], d[RPER], d1[RPER];
#pragma unroll
  for (int i = 0; i < RPER; ++i) {
    const int m = c.part + 8 * i;
    hv[i] = m < c.M ? to_f32(hd[m]) : 0.f;
    r1[i] = m < c.M ? round_as<E>(to_f32(r0[m]) + gm * hv[i]) : 0.f;
    d[i] = m < c.M ? dr[m] : 0.f;
  }
  rsa_bwd_row<E>(r1, d, c.M, c.part, d1);
  float part = 0.f;
  if (c.r < c.R) {
    E* dhd = reinterpret_cast<E*>(g.dhd) + ((int64_t)c.h * c.R + c.r) * c.M;
#pragma unroll
    for (int i = 0; i < RPER; ++i) {
      const int m = c.part + 8 * i;
      if (m < c.M) {
        dr[m] = d1[i];
        dhd[m] = from_f32<E>(round_as<E>(gm * d1[i]));
        part += d1[i] * hv[i];
      }
    }
  }
  for (int k = 32; k >= 1; k >>= 1) part += __shfl_xor(part, k);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = part;
  __syncthreads();
  if (threadIdx.x == 0)
    g.partials[((int64_t)c.tile * p.heads + c.h) * (2 + p.incoming)] = red[0] + red[1] + red[2] + red[3];
}

// ---------------------------------------------------------------- tiled products
// The bf16 route reader with widths that are multiples of 64 runs the row
// phases as their own kernels and each product as a tiled GEMM over all the
// rows of a head (128 rows x BN columns per workgroup, operands staged
// through LDS in 32-deep slabs, the weights read once per tile instead of
// once per 32 rows), with the element-wise work of the product fused into the
// epilogue.  The products are the fused kernel's, with the same operand and
// result roundings and the same contraction order (ascending 16-deep steps
// into one float32 accumulator), so both give the same bits.

__global__ __launch_bounds__(RNT) void route_rows16(gpa_route_problem p) {
  const int M = p.slots, R = p.batch * p.tokens;
  const RouteTile rtile = route_tile();
  const int h = rtile.h, row0 = rtile.tile * RR;
  __shared__ int row_b[RR], row_t[RR];
  const Rows rows = make_rows(row_b, row_t, row0, R, p.tokens);
  rows_r0_vec<bf16_t>(p, rows, row0, h, reinterpret_cast<bf16_t*>(p.r0) + (int64_t)h * R * M, nullptr, 0, 0);
}

constexpr int GM_BM = 128;           // rows per tile
constexpr int GM_KS = 32;            // contraction slab
constexpr int GM_LD = GM_KS + 8;     // LDS row pitch (bf16): 80 bytes
constexpr int GM_NT = 256;

// Row operand: element (h, r, k) at p + h * sh + r * sr + k.
struct RowOp {
  const bf16_t* p;
  int64_t sh, sr;
};
// One product: rows of `a` (K wide) times a packed weight b [H][nb][ldb]
// (output column n, contraction k contiguous: the layout route.py packs).
struct Prod {
  RowOp a;
  const bf16_t* b;
  int64_t nb, ldb;
  int K;
};
struct GemmShape {
  int R, N, H;
};

__device__ __forceinline__ float gelu_round(float x) { return round_as<bf16_t>(gelu(x)); }
typedef uint32_t u32x4n __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4n gelu_pack(u32x4n u) {
  float x[8];
  unpack_bf8(make_uint4(u.x, u.y, u.z, u.w), x);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = gelu_round(x[e]);
  const uint4 r = pack_bf8(x);
  return u32x4n{r.x, r.y, r.z, r.w};
}

// acc[rt][ct] += A(rows) B over one product; the workgroup's tile is rows
// row0 .. +127, columns col0 .. +BN-1 of head h; wave w computes rows
// 64 (w / 2) .. +63 and columns (BN / 2)(w % 2) .. as 32x32 MFMA tiles.
// GELU: the A operand is round(gelu(a)) of the stored rows.
template <int BN, bool GELU>
__device__ __forceinline__ void gemm_run(const Prod& pr, const GemmShape& sh, int h, int row0, int col0,
                                         bf16_t (*As)[GM_BM * GM_LD], bf16_t (*Bs)[BN * GM_LD],
                                         f32x16 (&acc)[2][BN / 64]) {
  constexpr int TN = BN / 64, BP = BN * GM_KS / 8 / GM_NT;  // B pieces per thread (2 or 1)
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, wr = w >> 1, wc = w & 1;
  const bf16_t* ap = pr.a.p + (int64_t)h * pr.a.sh;
  const bf16_t* bp = pr.b + (int64_t)h * pr.nb * pr.ldb + (int64_t)col0 * pr.ldb;
  // This thread's 16-byte pieces of each slab: A rows ar[i] (clamped to the
  // last row), B rows br[i]; column offsets kq.
  const bf16_t* ar[2];
  const bf16_t* br[BP];
  int alds[2], blds[BP];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int piece = tid + GM_NT * i, r = row0 + (piece >> 2);
    ar[i] = ap + (int64_t)(r < sh.R ? r : sh.R - 1) * pr.a.sr + 8 * (piece & 3);
    alds[i] = (piece >> 2) * GM_LD + 8 * (piece & 3);
  }
#pragma unroll
  for (int i = 0; i < BP; ++i) {
    const int piece = tid + GM_NT * i;
    br[i] = bp + (int64_t)(piece >> 2) * pr.ldb + 8 * (piece & 3);
    blds[i] = (piece >> 2) * GM_LD + 8 * (piece & 3);
  }
  const int steps = pr.K / GM_KS;
  // (register arrays of a native vector type: arrays of HIP's uint4 struct
  // are not always promoted to registers)
  u32x4n ra[2], rb[BP];
#pragma unroll
  for (int i = 0; i < 2; ++i) ra[i] = *reinterpret_cast<const u32x4n*>(ar[i]);
#pragma unroll
  for (int i = 0; i < BP; ++i) rb[i] = *reinterpret_cast<const u32x4n*>(br[i]);
  for (int s = 0; s < steps; ++s) {
    const int buf = s & 1;
#pragma unroll
    for (int i = 0; i < 2; ++i) *reinterpret_cast<u32x4n*>(&As[buf][alds[i]]) = GELU ? gelu_pack(ra[i]) : ra[i];
#pragma unroll
    for (int i = 0; i < BP; ++i) *reinterpret_cast<u32x4n*>(&Bs[buf][blds[i]]) = rb[i];
    __syncthreads();
    // the next slab's pieces (the last slab loads itself again, unused)
    const int kn = (s + 1 < steps ? s + 1 : s) * GM_KS;
#pragma unroll
    for (int i = 0; i < 2; ++i) ra[i] = *reinterpret_cast<const u32x4n*>(ar[i] + kn);
#pragma unroll
    for (int i = 0; i < BP; ++i) rb[i] = *reinterpret_cast<const u32x4n*>(br[i] + kn);
#pragma unroll
    for (int ks = 0; ks < GM_KS / 16; ++ks) {
      bf16x8 af[2], bf[TN];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
        af[rt] = *reinterpret_cast<const bf16x8*>(&As[buf][(64 * wr + 32 * rt + (lane & 31)) * GM_LD + 16 * ks +
                                                         8 * (lane >> 5)]);
#pragma unroll
      for (int ct = 0; ct < TN; ++ct)
        bf[ct] = *reinterpret_cast<const bf16x8*>(&Bs[buf][((BN / 2) * wc + 32 * ct + (lane & 31)) * GM_LD +
                                                           16 * ks + 8 * (lane >> 5)]);
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int ct = 0; ct < TN; ++ct) mma_bf16(acc[rt][ct], af[rt], bf[ct]);
    }
  }
  // every wave is done with the slabs before the caller reuses the LDS
  __syncthreads();
}

// Tile of a workgroup: heads slowest, so that each XCD serves a contiguous
// run of heads and keeps their weights in its L2.
struct GemmTile {
  int h, row0, col0;
};
template <int BN>
__device__ __forceinline__ GemmTile gemm_tile(const GemmShape& sh) {
  const int ntn = sh.N / BN, ntr = (sh.R + GM_BM - 1) / GM_BM, per_head = ntn * ntr;
  const int id = xcd_logical(blockIdx.x, gridDim.x);
  const int h = id / per_head, rem = id % per_head;
  return GemmTile{h, GM_BM * (rem / ntn), BN * (rem % ntn)};
}

// Eight consecutive bf16 / float32 values.
__device__ __forceinline__ void ld8(const bf16_t* p, float (&x)[8]) { unpack_bf8(*reinterpret_cast<const uint4*>(p), x); }
__device__ __forceinline__ void st8(bf16_t* p, const float (&x)[8]) { *reinterpret_cast<uint4*>(p) = pack_bf8(x); }
__device__ __forceinline__ void ld8(const float* p, float (&x)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}
__device__ __forceinline__ void st8(float* p, const float (&x)[8]) {
  *reinterpret_cast<f32x4*>(p) = f32x4{x[0], x[1], x[2], x[3]};
  *reinterpret_cast<f32x4*>(p + 4) = f32x4{x[4], x[5], x[6], x[7]};
}

// LDS of a product workgroup: the operand slabs, reused by the epilogue as a
// float32 staging tile of PR rows.
template <int BN>
struct GemmLds {
  static constexpr int PR = BN <= 128 ? 64 : 32, LDT = BN + 4;
  static constexpr int SLABS = 2 * (GM_BM + BN) * GM_LD * 2, STAGE = PR * LDT * 4;
  static constexpr int BYTES = SLABS > STAGE ? SLABS : STAGE;
};

// The epilogue: Epi::combine(acc, acc2) per element in registers; then, PR
// rows at a time, the values go through LDS so that every thread handles
// whole 8-column row pieces: pre = epi.load(h, r, c) for all of a thread's
// pieces first, then epi.store(h, r, c, v, pre, epi.head(h)), whose return
// values summed over each 32-row block go to epi.block_sum (Epi::kPart).
template <int BN, bool GELU, bool DUAL, typename Epi>
__global__ __launch_bounds__(GM_NT) void route_gemm16(Prod p1, Prod p2, GemmShape sh, Epi epi) {
  constexpr int TN = BN / 64, PR = GemmLds<BN>::PR, LDT = GemmLds<BN>::LDT;
  constexpr int VPR = BN / 8, NVT = PR * VPR / GM_NT;  // pieces per row, per thread and pass
  __shared__ __align__(16) unsigned char smem[GemmLds<BN>::BYTES];
  auto As = reinterpret_cast<bf16_t(*)[GM_BM * GM_LD]>(smem);
  auto Bs = reinterpret_cast<bf16_t(*)[BN * GM_LD]>(smem + 2 * GM_BM * GM_LD * 2);
  float* stage = reinterpret_cast<float*>(smem);
  const GemmTile t = gemm_tile<BN>(sh);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, wr = w >> 1, wc = w & 1;
  f32x16 acc[2][TN], acc2[2][TN];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int ct = 0; ct < TN; ++ct) acc[rt][ct] = acc2[rt][ct] = f32x16{};
  gemm_run<BN, GELU>(p1, sh, t.h, t.row0, t.col0, As, Bs, acc);
  if constexpr (DUAL) gemm_run<BN, false>(p2, sh, t.h, t.row0, t.col0, As, Bs, acc2);
  const float hs = epi.head(t.h);
  __shared__ float red[GM_NT / 64][2];
#pragma unroll
  for (int pass = 0; pass < GM_BM / PR; ++pass) {
    // the 32-row tiles of this pass: rows 64 wr + 32 rt in [pass PR, pass PR + PR)
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int rbase = 64 * wr + 32 * rt - pass * PR;
      if (rbase >= 0 && rbase < PR) {
#pragma unroll
        for (int ct = 0; ct < TN; ++ct)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            stage[(rbase + acc_row(i, lane >> 5)) * LDT + (BN / 2) * wc + 32 * ct + (lane & 31)] =
                epi.combine(acc[rt][ct][i], acc2[rt][ct][i]);
      }
    }
    __syncthreads();
    typename Epi::Pre pre[NVT];
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
      const int v = tid + GM_NT * j, r = t.row0 + pass * PR + v / VPR;
      pre[j] = epi.load(t.h, r < sh.R ? r : t.row0, t.col0 + 8 * (v % VPR));  // the tile's first row is valid
    }
    float part0 = 0.f, part1 = 0.f;  // rows below / from 32 of the pass (registers, not a private array)
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
      const int v = tid + GM_NT * j, row = v / VPR, r = t.row0 + pass * PR + row;
      float x[8];
      ld8(stage + row * LDT + 8 * (v % VPR), x);
      if (r < sh.R) {
        const float y = epi.store(t.h, r, t.col0 + 8 * (v % VPR), x, pre[j], hs);
        if (row < 32) part0 += y;
        else part1 += y;
      }
    }
    if constexpr (Epi::kPart) {
      // A tile spans all N columns (BN == N), so a block's sum is complete here.
#pragma unroll
      for (int k = 0; k < PR / 32; ++k) {
        float x = k ? part1 : part0;
        for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
        if (lane == 0) red[w][k] = x;
      }
    }
    __syncthreads();
    if constexpr (Epi::kPart) {
      if (tid < PR / 32) {
        const int r0 = t.row0 + pass * PR + 32 * tid;
        if (r0 < sh.R) epi.block_sum(t.h, r0 / RR, red[0][tid] + red[1][tid] + red[2][tid] + red[3][tid]);
      }
    }
  }
}

// h1 = round(r0 U), saved.
struct EpiH1 {
  static constexpr bool kPart = false;
  bf16_t* h1;
  int64_t sh, sr;
  typedef int Pre;
  __device__ float head(int) const { return 0.f; }
  __device__ float combine(float a, float) const { return a; }
  __device__ Pre load(int, int, int) const { return 0; }
  __device__ float store(int h, int r, int c, const float (&v)[8], Pre, float) const {
    st8(h1 + h * sh + r * sr + c, v);
    return 0.f;
  }
  __device__ void block_sum(int, int, float) const {}
};
// hd = round(gelu(h1) D), saved; r1 = round(r0 + mlp_gain hd), the route output.
struct EpiHd {
  static constexpr bool kPart = false;
  bf16_t* hd;
  const bf16_t* r0;
  int64_t sh, sr;  // of hd and r0: [H][R][M]
  const float* mlp_gain;
  bf16_t* route;
  int64_t route_sh, route_sr;
  typedef uint4 Pre;
  __device__ float head(int h) const { return mlp_gain[h]; }
  __device__ float combine(float a, float) const { return round_as<bf16_t>(a); }
  __device__ Pre load(int h, int r, int c) const { return *reinterpret_cast<const uint4*>(r0 + h * sh + r * sr + c); }
  __device__ float store(int h, int r, int c, const float (&d)[8], Pre r0v, float g) const {
    st8(hd + h * sh + r * sr + c, d);
    float x[8];
    unpack_bf8(r0v, x);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] += g * d[j];
    st8(route + h * route_sh + r * route_sr + c, x);
    return 0.f;
  }
  __device__ void block_sum(int, int, float) const {}
};
// qo = round(round(r1 W_rs) + round(query_scale round(q W_qs))).
struct EpiQo {
  static constexpr bool kPart = false;
  bf16_t* qo;
  int64_t sh, sr;
  float query_scale;
  typedef int Pre;
  __device__ float head(int) const { return 0.f; }
  __device__ float combine(float a, float a2) const {
    return round_as<bf16_t>(a) + round_as<bf16_t>(query_scale * round_as<bf16_t>(a2));
  }
  __device__ Pre load(int, int, int) const { return 0; }
  __device__ float store(int h, int r, int c, const float (&v)[8], Pre, float) const {
    st8(qo + h * sh + r * sr + c, v);
    return 0.f;
  }
  __device__ void block_sum(int, int, float) const {}
};

// balanced_bridge: qr = round(r1 W_rs) and qdir = round(query_scale round(q W_qs))
// saved separately (rows [H][R][M]), each by a product of its own;
// route_mix_fwd forms qo from them.
struct EpiQr {
  static constexpr bool kPart = false;
  bf16_t* qr;
  int64_t sh, sr;
  typedef int Pre;
  __device__ float head(int) const { return 0.f; }
  __device__ float combine(float a, float) const { return a; }
  __device__ Pre load(int, int, int) const { return 0; }
  __device__ float store(int h, int r, int c, const float (&v)[8], Pre, float) const {
    st8(qr + h * sh + r * sr + c, v);
    return 0.f;
  }
  __device__ void block_sum(int, int, float) const {}
};
struct EpiQdir {
  static constexpr bool kPart = false;
  bf16_t* qdir;
  int64_t sh, sr;
  float query_scale;
  typedef int Pre;
  __device__ float head(int) const { return 0.f; }
  __device__ float combine(float a, float) const { return round_as<bf16_t>(query_scale * round_as<bf16_t>(a)); }
  __device__ Pre load(int, int, int) const { return 0; }
  __device__ float store(int h, int r, int c, const float (&v)[8], Pre, float) const {
    st8(qdir + h * sh + r * sr + c, v);
    return 0.f;
  }
  __device__ void block_sum(int, int, float) const {}
};

// Backward.  d r1 = round(dqo W_rs^T) (+ d route, rounded) is kept in the
// float32 d base buffer until the row kernel overwrites it; d hd = round(mlp_gain
// d r1) and round(query_scale dqo) are saved rows; each 32-row block's
// sum of d r1 . hd is d mlp_gain's partial.
// With balanced_bridge the W_rs product reads the gradient of qr and the
// q W_qs gradient comes from that of qdir (dqo below, rows [H][R][M]).  With
// rsa_update the product's result is the gradient of the rescaled row: it is
// stored alone (d r1', rounded) and route_rsa_bwd finishes d r1, d hd and the
// partial sums.
struct EpiDr1 {
  static constexpr bool kPart = true;
  const bf16_t* dqo;
  const bf16_t* droute;  // may be null
  int64_t io_sh, io_sr;  // d route rows ([B,T,H,M], uniformly strided)
  int64_t dq_sh, dq_sr;  // dqo rows
  int rsa;
  const bf16_t* hd;
  bf16_t *dhd, *dqs;
  int64_t sh, sr;        // hd, dhd, dqs: [H][R][M]
  float* dr1;            // d base [B,T,H,M] float32
  int64_t dr_sh, dr_sr;
  const float* mlp_gain;
  float query_scale;
  float* partials;       // [R / 32][H][2 + incoming], slot 0
  int heads, nparts;
  struct Pre {
    uint4 dro, hd, dqo;
  };
  __device__ float head(int h) const { return mlp_gain[h]; }
  __device__ float combine(float a, float) const { return round_as<bf16_t>(a); }
  __device__ Pre load(int h, int r, int c) const {
    const uint4 z = make_uint4(0, 0, 0, 0);
    return Pre{droute ? *reinterpret_cast<const uint4*>(droute + h * io_sh + r * io_sr + c) : z,
               *reinterpret_cast<const uint4*>(hd + h * sh + r * sr + c),
               *reinterpret_cast<const uint4*>(dqo + h * dq_sh + r * dq_sr + c)};
  }
  __device__ float store(int h, int r, int c, const float (&v)[8], const Pre& x, float gm) const {
    float d[8], dro[8], hv[8], dq[8], dh[8];
    unpack_bf8(x.dro, dro);
    unpack_bf8(x.hd, hv);
    unpack_bf8(x.dqo, dq);
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      d[j] = droute ? round_as<bf16_t>(v[j] + dro[j]) : v[j];
      dh[j] = gm * d[j];
      dq[j] *= query_scale;
      part += d[j] * hv[j];
    }
    const int64_t o = h * sh + r * sr + c;
    if (!rsa) st8(dhd + o, dh);
    st8(dqs + o, dq);
    st8(dr1 + h * dr_sh + r * dr_sr + c, d);
    return rsa ? 0.f : part;
  }
  __device__ void block_sum(int h, int blk, float x) const { partials[((int64_t)blk * heads + h) * nparts] = x; }
};
// d h1 = round(round(d hd D^T) gelu'(h1)), and round(gelu(h1)) for the weight
// gradients (it shares gelu'(h1)'s erf).
struct EpiDh1 {
  static constexpr bool kPart = false;
  const bf16_t* h1;
  bf16_t *dh1, *hg;
  int64_t sh, sr;  // [H][R][2M]
  typedef uint4 Pre;
  __device__ float head(int) const { return 0.f; }
  __device__ float combine(float a, float) const { return round_as<bf16_t>(a); }
  __device__ Pre load(int h, int r, int c) const { return *reinterpret_cast<const uint4*>(h1 + h * sh + r * sr + c); }
  __device__ float store(int h, int r, int c, const float (&v)[8], Pre hv, float) const {
    float x[8], d[8], gl[8];
    unpack_bf8(hv, x);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      d[j] = v[j] * gelu_grad(x[j]);
      gl[j] = gelu(x[j]);
    }
    const int64_t o = h * sh + r * sr + c;
    st8(dh1 + o, d);
    st8(hg + o, gl);
    return 0.f;
  }
  __device__ void block_sum(int, int, float) const {}
};
// d r0 = round(d r1 + round(d h1 U^T)), in place of d r1.
struct EpiDr0 {
  static constexpr bool kPart = false;
  float* dr;
  int64_t sh, sr;
  struct Pre {
    float x[8];
  };
  __device__ float head(int) const { return 0.f; }
  __device__ float combine(float a, float) const { return round_as<bf16_t>(a); }
  __device__ Pre load(int h, int r, int c) const {
    Pre p;
    ld8(dr + h * sh + r * sr + c, p.x);
    return p;
  }
  __device__ float store(int h, int r, int c, const float (&v)[8], const Pre& d1, float) const {
    float y[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) y[j] = round_as<bf16_t>(d1.x[j] + v[j]);
    st8(dr + h * sh + r * sr + c, y);
    return 0.f;
  }
  __device__ void block_sum(int, int, float) const {}
};
// d q = round(round(query_scale dqo) W_qs^T).
struct EpiDq {
  static constexpr bool kPart = false;
  bf16_t* dq;
  int64_t sh, sr;
  typedef int Pre;
  __device__ float head(int) const { return 0.f; }
  __device__ float combine(float a, float) const { return a; }
  __device__ Pre load(int, int, int) const { return 0; }
  __device__ float store(int h, int r, int c, const float (&v)[8], Pre, float) const {
    st8(dq + h * sh + r * sr + c, v);
    return 0.f;
  }
  __device__ void block_sum(int, int, float) const {}
};

// Row backward of the tiled path: d r0 from the d base buffer (float32,
// written by the products), then rows_bwd_vec; partial slots 1 and 2 + e.
__global__ __launch_bounds__(RNT) void route_rows16_bwd(gpa_route_problem p, gpa_route_grads g) {
  __shared__ float red[RW][1 + GPA_ROUTE_MAX_INCOMING];
  const int M = p.slots, R = p.batch * p.tokens, H = p.heads, NI = p.incoming;
  const RouteTile rtile = route_tile();
  const int h = rtile.h, row0 = rtile.tile * RR, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __shared__ int row_b[RR], row_t[RR];
  const Rows rows = make_rows(row_b, row_t, row0, R, p.tokens);
  const int c = 8 * (tid & 31), rsub = tid >> 5, cc = c < M ? c : 0;
  float d0v[VPASS][8];
#pragma unroll
  for (int i = 0; i < VPASS; ++i) {
    const int r = row0 + rsub + 8 * i, rr = r < R ? r : R - 1;
    const float* src = reinterpret_cast<const float*>(g.dbase.ptr) + rows.at(g.dbase, rr, h) + cc;
    const f32x4 a = *reinterpret_cast<const f32x4*>(src), b = *reinterpret_cast<const f32x4*>(src + 4);
    d0v[i][0] = a.x; d0v[i][1] = a.y; d0v[i][2] = a.z; d0v[i][3] = a.w;
    d0v[i][4] = b.x; d0v[i][5] = b.y; d0v[i][6] = b.z; d0v[i][7] = b.w;
  }
  // every lane has its d r0 values before any row of the workgroup is overwritten
  __syncthreads();
  float part_gain = 0.f, part_w[GPA_ROUTE_MAX_INCOMING] = {0.f, 0.f, 0.f};
  rows_bwd_vec<bf16_t>(p, g, rows, row0, h, d0v, part_gain, part_w);
  float vals[1 + GPA_ROUTE_MAX_INCOMING] = {part_gain, part_w[0], part_w[1], part_w[2]};
#pragma unroll
  for (int k = 0; k < 1 + GPA_ROUTE_MAX_INCOMING; ++k) {
    float x = vals[k];
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
    if (lane == 0) red[wave][k] = x;
  }
  __syncthreads();
  if (tid < 1 + NI) {
    float x = 0.f;
    for (int w = 0; w < RW; ++w) x += red[w][tid];
    g.partials[((int64_t)rtile.tile * H + h) * (2 + NI) + 1 + tid] = x;
  }
}

template <typename E, bool VEC>
__global__ __launch_bounds__(RNT) void route_bwd(gpa_route_problem p, gpa_route_grads g) {
  using W = typename Wt<E>::type;
  HIP_DYNAMIC_SHARED(float, lds)
  __shared__ float red[RW][2 + GPA_ROUTE_MAX_INCOMING];
  const int M = p.slots, Dk = p.key_dim, R = p.batch * p.tokens, H = p.heads, NI = p.incoming;
  const RouteTile rtile = route_tile();
  const int h = rtile.h, row0 = rtile.tile * RR;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kM = pad16(M), k2M = pad16(2 * M);
  const int lda = kM + 4, ldh = k2M + 4;
  float* G = lds;                // dqo, then round(qs dqo)   [RR][lda]
  float* A2 = lds + RR * lda;    // d hd, then d r0           [RR][lda]
  float* H2 = A2 + RR * lda;     // d h1                      [RR][ldh]
  __shared__ int row_b[RR], row_t[RR];
  const Rows rows = make_rows(row_b, row_t, row0, R, p.tokens);
  const E* sh1 = reinterpret_cast<const E*>(p.h1) + (int64_t)h * R * 2 * M;
  const E* shd = reinterpret_cast<const E*>(p.hd) + (int64_t)h * R * M;
  E* gdh1 = reinterpret_cast<E*>(g.dh1) + (int64_t)h * R * 2 * M;
  E* ghg = reinterpret_cast<E*>(g.hg) + (int64_t)h * R * 2 * M;
  E* gdhd = reinterpret_cast<E*>(g.dhd) + (int64_t)h * R * M;
  E* gdqs = reinterpret_cast<E*>(g.dqs) + (int64_t)h * R * M;
  float part_mg = 0.f, part_gain = 0.f, part_w[GPA_ROUTE_MAX_INCOMING] = {0.f, 0.f, 0.f};

  // ---- dqo (balanced: the gradient of qr) -> G
  const gpa_operand& d1src = p.balanced ? g.dqr : g.dqo;
  if constexpr (VEC) {
    const int c = 8 * (tid & 31), rsub = tid >> 5;
    uint4 dv[VPASS];
#pragma unroll
    for (int i = 0; i < VPASS; ++i) {
      const int r = row0 + rsub + 8 * i;
      dv[i] = (c < M && r < R) ? *reinterpret_cast<const uint4*>(reinterpret_cast<const bf16_t*>(d1src.ptr) +
                                                                  rows.at(d1src, r, h) + c)
                               : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < VPASS; ++i) {
      const int row = rsub + 8 * i;
      float x[8];
      unpack_bf8(dv[i], x);
      if (c < kM) {
        *reinterpret_cast<f32x4*>(&G[row * lda + c]) = f32x4{x[0], x[1], x[2], x[3]};
        *reinterpret_cast<f32x4*>(&G[row * lda + c + 4]) = f32x4{x[4], x[5], x[6], x[7]};
      }
    }
  } else {
    const int row = tid >> 3, part = tid & 7, r = row0 + row;
    const bool valid = r < R;
    const E* dqo = reinterpret_cast<const E*>(d1src.ptr) + rows.at(d1src, valid ? r : R - 1, h);
#pragma unroll
    for (int i = 0; i < RPER; ++i) {
      const int m = part + 8 * i;
      if (m < kM) G[row * lda + m] = (valid && m < M) ? to_f32(dqo[m]) : 0.f;
    }
  }
  __syncthreads();

  // ---- d r1 = dqo W_rs^T (+ d route); d hd = mlp_gain d r1 -> A2
  f32x16 dr1[RTMAX];
  {
    const W* rs = reinterpret_cast<const W*>(p.rs) + (int64_t)h * pad32(M) * kM;
    const float gm = p.mlp_gain[h];
    const E* droute = reinterpret_cast<const E*>(g.droute.ptr);
#pragma unroll
    for (int s = 0; s < RTMAX; ++s) {
      const int t = wave + RW * s;
      dr1[s] = f32x16{};
      if (t >= pad32(M) / 32) continue;
      f32x16 acc = {};
      tile_gemm(acc, G, lda, rs, kM, kM, 32 * t, lane);
      // The row operands are all loaded (at clamped addresses) before the
      // first store, so that their latencies overlap.
      // Without d route the same loads read the saved hd rows (always valid).
      float dro[16], hdv[16];
      const E* drp = droute ? droute : shd;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int col = 32 * t + (lane & 31), r = row0 + acc_row(i, lane >> 5);
        // Masked entries read the tile's first row (rows.at only knows this
        // tile's rows; row0 < R always).
        const bool ok = col < M && r < R;
        const int rc = ok ? r : row0, cc = ok ? col : 0;
        dro[i] = to_f32(drp[droute ? rows.at(g.droute, rc, h) + cc : (int64_t)rc * M + cc]);
        hdv[i] = to_f32(shd[(int64_t)rc * M + cc]);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = acc_row(i, lane >> 5), col = 32 * t + (lane & 31), r = row0 + row;
        if (col < M) {
          float d = round_as<E>(acc[i]);
          if (droute && r < R) d = round_as<E>(d + dro[i]);
          if (r >= R) d = 0.f;
          dr1[s][i] = d;
          if (p.rsa) {  // the gradient of the rescaled row; rsa_update's backward follows
            A2[row * lda + col] = d;
            continue;
          }
          const float dhd = round_as<E>(gm * d);
          A2[row * lda + col] = dhd;
          if (r < R) {
            part_mg += d * hdv[i];
            gdhd[(int64_t)r * M + col] = from_f32<E>(dhd);
          }
        } else if (col < kM) {
          A2[row * lda + col] = 0.f;
        }
      }
    }
  }
  __syncthreads();

  // ---- rsa_update: d r1 from d r1' (A2) and the recomputed r1; then d hd -> A2
  if (p.rsa) {
    {
      const int row = tid >> 3, part = tid & 7, r = row0 + row, rc = r < R ? r : R - 1;
      const E* r0v = reinterpret_cast<const E*>(p.r0) + ((int64_t)h * R + rc) * M;
      const float gm = p.mlp_gain[h];
      float r1[RPER], d[RPER], d1[RPER];
#pragma unroll
      for (int i = 0; i < RPER; ++i) {
        const int m = part + 8 * i;
        r1[i] = m < M ? round_as<E>(to_f32(r0v[m]) + gm * to_f32(shd[(int64_t)rc * M + m])) : 0.f;
        d[i] = m < M ? A2[row * lda + m] : 0.f;
      }
      rsa_bwd_row<E>(r1, d, M, part, d1);
#pragma unroll
      for (int i = 0; i < RPER; ++i)
        if (part + 8 * i < M) A2[row * lda + part + 8 * i] = r < R ? d1[i] : 0.f;
    }
    __syncthreads();
    const float gm = p.mlp_gain[h];
#pragma unroll
    for (int s = 0; s < RTMAX; ++s) {
      const int t = wave + RW * s;
      if (t >= pad32(M) / 32) continue;
      float hdv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int col = 32 * t + (lane & 31), r = row0 + acc_row(i, lane >> 5);
        const bool ok = col < M && r < R;
        hdv[i] = to_f32(shd[(int64_t)(ok ? r : row0) * M + (ok ? col : 0)]);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = acc_row(i, lane >> 5), col = 32 * t + (lane & 31), r = row0 + row;
        if (col < M) {
          const float d = A2[row * lda + col];
          dr1[s][i] = d;
          const float dhd = round_as<E>(gm * d);
          A2[row * lda + col] = dhd;
          if (r < R) {
            part_mg += d * hdv[i];
            gdhd[(int64_t)r * M + col] = from_f32<E>(dhd);
          }
        }
      }
    }
    __syncthreads();
  }

  // ---- G <- round(query_scale dqo) (the gradient of q W_qs; balanced: of ddir)
  if constexpr (VEC) {
    const int c = 8 * (tid & 31), rsub = tid >> 5;
    if (c < M) {
#pragma unroll
      for (int i = 0; i < VPASS; ++i) {
        const int row = rsub + 8 * i, r = row0 + row;
        float* gr = &G[row * lda + c];
        float x[8];
        if (p.balanced) {
          const uint4 u = r < R ? *reinterpret_cast<const uint4*>(reinterpret_cast<const bf16_t*>(g.ddir.ptr) +
                                                                  rows.at(g.ddir, r, h) + c)
                                : make_uint4(0, 0, 0, 0);
          unpack_bf8(u, x);
        } else {
          const f32x4 a = *reinterpret_cast<const f32x4*>(gr), b = *reinterpret_cast<const f32x4*>(gr + 4);
          x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = round_as<E>(p.query_scale * x[e]);
        *reinterpret_cast<f32x4*>(gr) = f32x4{x[0], x[1], x[2], x[3]};
        *reinterpret_cast<f32x4*>(gr + 4) = f32x4{x[4], x[5], x[6], x[7]};
        if (r < R) *reinterpret_cast<uint4*>(gdqs + (int64_t)r * M + c) = pack_bf8(x);
      }
    }
  } else {
    const int row = tid >> 3, part = tid & 7, r = row0 + row;
    const E* ddir = p.balanced ? reinterpret_cast<const E*>(g.ddir.ptr) + rows.at(g.ddir, r < R ? r : R - 1, h)
                               : nullptr;
#pragma unroll
    for (int i = 0; i < RPER; ++i) {
      const int m = part + 8 * i;
      if (m < M) {
        const float src = ddir ? (r < R ? to_f32(ddir[m]) : 0.f) : G[row * lda + m];
        const float x = round_as<E>(p.query_scale * src);
        G[row * lda + m] = x;
        if (r < R) gdqs[(int64_t)r * M + m] = from_f32<E>(x);
      }
    }
  }

  // ---- d h1 = (d hd D^T) gelu'(h1) -> H2
  {
    const W* down = reinterpret_cast<const W*>(p.down) + (int64_t)h * pad32(2 * M) * kM;
    for (int t = wave; t < pad32(2 * M) / 32; t += RW) {
      f32x16 acc = {};
      tile_gemm(acc, A2, lda, down, kM, kM, 32 * t, lane);
      float h1v[16];  // loaded before the first store (see above)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int col = 32 * t + (lane & 31), r = row0 + acc_row(i, lane >> 5);
        const bool ok = col < 2 * M && r < R;
        h1v[i] = to_f32(sh1[(int64_t)(ok ? r : 0) * 2 * M + (ok ? col : 0)]);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = acc_row(i, lane >> 5), col = 32 * t + (lane & 31), r = row0 + row;
        if (col < 2 * M) {
          float d = 0.f;
          if (r < R) {
            const float x = h1v[i];
            d = round_as<E>(round_as<E>(acc[i]) * gelu_grad(x));
            gdh1[(int64_t)r * 2 * M + col] = from_f32<E>(d);
            ghg[(int64_t)r * 2 * M + col] = from_f32<E>(gelu(x));  // shares gelu_grad's erf
          }
          H2[row * ldh + col] = d;
        } else if (col < k2M) {
          H2[row * ldh + col] = 0.f;
        }
      }
    }
  }
  __syncthreads();

  // ---- d r0 = d r1 + d h1 U^T -> A2;  d q = round(qs dqo) W_qs^T
  {
    const W* up = reinterpret_cast<const W*>(p.up) + (int64_t)h * pad32(M) * k2M;
#pragma unroll
    for (int s = 0; s < RTMAX; ++s) {
      const int t = wave + RW * s;
      if (t >= pad32(M) / 32) continue;
      f32x16 acc = {};
      tile_gemm(acc, H2, ldh, up, k2M, k2M, 32 * t, lane);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = acc_row(i, lane >> 5), col = 32 * t + (lane & 31);
        if (col < M) A2[row * lda + col] = round_as<E>(dr1[s][i] + round_as<E>(acc[i]));
      }
    }
    const W* qs = reinterpret_cast<const W*>(p.qs) + (int64_t)h * pad32(Dk) * kM;
    E* dq = reinterpret_cast<E*>(g.dq.ptr);
    for (int t = wave; t < pad32(Dk) / 32; t += RW) {
      f32x16 acc = {};
      tile_gemm(acc, G, lda, qs, kM, kM, 32 * t, lane);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = acc_row(i, lane >> 5), col = 32 * t + (lane & 31), r = row0 + row;
        if (col < Dk && r < R) dq[rows.at(g.dq, r, h) + col] = from_f32<E>(round_as<E>(acc[i]));
      }
    }
  }
  __syncthreads();

  // ---- softmax and relation-read backward of each row
  if constexpr (VEC) {
    const int c = 8 * (tid & 31), rsub = tid >> 5;
    float d0v[VPASS][8];
#pragma unroll
    for (int i = 0; i < VPASS; ++i) {
      const int row = rsub + 8 * i;
      const f32x4 a = *reinterpret_cast<const f32x4*>(&A2[row * lda + (c < M ? c : 0)]);
      const f32x4 b = *reinterpret_cast<const f32x4*>(&A2[row * lda + (c < M ? c : 0) + 4]);
      d0v[i][0] = a.x; d0v[i][1] = a.y; d0v[i][2] = a.z; d0v[i][3] = a.w;
      d0v[i][4] = b.x; d0v[i][5] = b.y; d0v[i][6] = b.z; d0v[i][7] = b.w;
    }
    rows_bwd_vec<E>(p, g, rows, row0, h, d0v, part_gain, part_w);
  } else {
    const int row = tid >> 3, part = tid & 7, r = row0 + row;
    const bool valid = r < R;
    const int rc = valid ? r : R - 1;
    float v[RPER], z[RPER], pr[RPER], inv;
    row_base<E>(p, rows, rc, h, part, v, z, inv);
    row_softmax<E>(M, part, v, pr);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < RPER; ++i)
      if (part + 8 * i < M) s += pr[i] * A2[row * lda + part + 8 * i];
    s = sum8(s);
    float* dbase = reinterpret_cast<float*>(g.dbase.ptr) + rows.at(g.dbase, rc, h);
#pragma unroll
    for (int i = 0; i < RPER; ++i) {
      const int m = part + 8 * i;
      // d base' (the softmax input) overwrites v
      v[i] = m < M ? pr[i] * (A2[row * lda + m] - s) : 0.f;
      if (valid && m < M) dbase[m] = v[i];
    }
    if (NI > 0) {
      const float gain = p.gain[h];
      float dz[RPER], szz = 0.f;
#pragma unroll
      for (int i = 0; i < RPER; ++i) {
        const int m = part + 8 * i;
        const float th = tanhf(z[i]);
        if (valid && m < M) part_gain += v[i] * th;
        dz[i] = m < M ? gain * v[i] * (1.f - th * th) : 0.f;
        szz += dz[i] * z[i];
      }
      const float mzz = sum8(szz) / M;
      float sc = 0.f;
#pragma unroll
      for (int i = 0; i < RPER; ++i) {
        dz[i] = part + 8 * i < M ? (dz[i] - z[i] * mzz) * inv : 0.f;  // d centred
        sc += dz[i];
      }
      const float mc = sum8(sc) / M;
#pragma unroll
      for (int i = 0; i < RPER; ++i) dz[i] -= mc;  // d incoming
      for (int e = 0; e < NI; ++e) {
        const float w = p.edge_weight[e * H + h];
        const E* msg = reinterpret_cast<const E*>(p.msg[e].ptr) + rows.at(p.msg[e], rc, h);
        E* dmsg = reinterpret_cast<E*>(g.dmsg[e].ptr) + rows.at(g.dmsg[e], rc, h);
        float sw = 0.f;
#pragma unroll
        for (int i = 0; i < RPER; ++i) {
          const int m = part + 8 * i;
          if (m < M) {
            sw += dz[i] * to_f32(msg[m]);
            if (valid) dmsg[m] = from_f32<E>(round_as<E>(w * dz[i]));
          }
        }
        if (valid) part_w[e] += sw;
      }
    }
  }

  // ---- per-block sums of the scalar gradients
  {
    float vals[2 + GPA_ROUTE_MAX_INCOMING] = {part_mg, part_gain, part_w[0], part_w[1], part_w[2]};
#pragma unroll
    for (int k = 0; k < 2 + GPA_ROUTE_MAX_INCOMING; ++k) {
      float x = vals[k];
      for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
      if (lane == 0) red[wave][k] = x;
    }
    __syncthreads();
    if (tid < 2 + NI) {
      float x = 0.f;
      for (int w = 0; w < RW; ++w) x += red[w][tid];
      g.partials[((int64_t)rtile.tile * H + h) * (2 + NI) + tid] = x;
    }
  }
}

// Weight gradients C[h][i][j] = sum_r A[h][r][i] B[h][r][j] over the R rows.
// A workgroup owns a 64x64 tile of C (a 32x32 quadrant per wave) and a span
// of WKC rows; slabs of 32 rows of A and B are read with 16-byte loads,
// stored transposed in LDS, and fed to MFMA; the spans' partial tiles are
// added into C (cleared first) with float atomics and rounded at the end.
struct TnOperand {
  const void* ptr;
  int64_t rs, hs;  // row and head strides (elements)
  int width;
};

constexpr int WT = 64;     // output tile
constexpr int WK = 32;     // rows per slab
constexpr int WP = WK + 1; // LDS pitch (floats)
constexpr int WKC = 256;   // rows per workgroup

template <typename E>
__device__ __forceinline__ void load8(const TnOperand& o, int h, int r, int c, int rend, float (&x)[8]) {
#pragma unroll
  for (int s = 0; s < 8; ++s) x[s] = 0.f;
  if (r >= rend) return;
  const E* p = reinterpret_cast<const E*>(o.ptr) + (int64_t)h * o.hs + (int64_t)r * o.rs + c;
  if (c + 8 <= o.width && (reinterpret_cast<uintptr_t>(p) & 15) == 0) {
    if constexpr (std::is_same<E, float>::value) {
      const f32x4 u = reinterpret_cast<const f32x4*>(p)[0], v = reinterpret_cast<const f32x4*>(p)[1];
      x[0] = u.x; x[1] = u.y; x[2] = u.z; x[3] = u.w; x[4] = v.x; x[5] = v.y; x[6] = v.z; x[7] = v.w;
    } else {
      const uint4 w = *reinterpret_cast<const uint4*>(p);
      const unsigned ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        x[2 * s] = __uint_as_float(ws[s] << 16);
        x[2 * s + 1] = __uint_as_float(ws[s] & 0xffff0000u);
      }
    }
  } else {
#pragma unroll
    for (int s = 0; s < 8; ++s)
      if (c + s < o.width) x[s] = to_f32(p[s]);
  }
}

template <typename E>
__global__ __launch_bounds__(RNT) void route_wgrad(TnOperand a, TnOperand b, float* c, int R) {
  __shared__ float As[WT][WP], Bs[WT][WP];
  const int h = blockIdx.y, tj = (b.width + WT - 1) / WT;
  const int i0 = WT * (blockIdx.x / tj), j0 = WT * (blockIdx.x % tj);
  const int rbeg = blockIdx.z * WKC, rend = rbeg + WKC < R ? rbeg + WKC : R;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wi = (wave & 1) * 32 + (lane & 31), wj = (wave >> 1) * 32 + (lane & 31);
  const int lr = tid >> 3, lc = (tid & 7) * 8;
  f32x16 acc = {};
  for (int k0 = rbeg; k0 < rend; k0 += WK) {
    float xa[8], xb[8];
    load8<E>(a, h, k0 + lr, i0 + lc, rend, xa);
    load8<E>(b, h, k0 + lr, j0 + lc, rend, xb);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      As[lc + s][lr] = xa[s];
      Bs[lc + s][lr] = xb[s];
    }
    __syncthreads();
    if constexpr (std::is_same<E, float>::value) {
#pragma unroll
      for (int kk = 0; kk < WK; kk += 8) {
        const int k = kk + 4 * (lane >> 5);
        mma8(acc, f32x4{As[wi][k], As[wi][k + 1], As[wi][k + 2], As[wi][k + 3]},
             f32x4{Bs[wj][k], Bs[wj][k + 1], Bs[wj][k + 2], Bs[wj][k + 3]});
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < WK; kk += 16) {
        const int k = kk + 8 * (lane >> 5);
        bf16x8 av, bv;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          av[s] = (__bf16)As[wi][k + s];
          bv[s] = (__bf16)Bs[wj][k + s];
        }
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int i = i0 + (wave & 1) * 32 + acc_row(r, lane >> 5), j = j0 + wj;
    if (i < a.width && j < b.width) atomicAdd(&c[((int64_t)h * a.width + i) * b.width + j], acc[r]);
  }
}

__global__ void fill_zero(float* c, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    c[i] = 0.f;
}
template <typename E>
__global__ void round_in_place(float* c, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    c[i] = round_as<E>(c[i]);
}

// bf16 weight gradients, all four products in one launch.  A workgroup owns
// a 128x128 tile of one product's C for one head and a span of rows; the
// span is walked in slabs of 64 rows.  Waves 0-1 stage A, waves 2-3 stage B:
// each lane reads an 8x8 block (8 rows of 16 bytes), transposes it in
// registers and writes its 8 columns to LDS as 16-byte rows of 8 tokens, so
// that LDS holds [column][token] and each MFMA operand is one 16-byte read.
// With a 72-element pitch and lanes ordered row block first, the writes and
// the reads both touch 16 distinct 4-bank groups per 16 lanes.  Partial tiles
// of the spans are added into C (cleared first) with float atomics.
constexpr int GT = 128;         // output tile
constexpr int GK = 64;          // rows per slab
constexpr int GP = GK + 8;      // LDS pitch (bf16)
constexpr int GNT = 256;
constexpr int G_WGS = 512;      // workgroups the row spans aim for
constexpr size_t G_LDS = 2 * GT * GP * sizeof(uint16_t);  // A and B slabs

struct WJob {
  TnOperand a, b;
  float* c;
  int tj, tiles;  // column tiles of C, tiles of C
};
struct WJobs {
  WJob j0, j1, j2, j3;
  int span, R, tiles, heads, n;  // tiles of all four products, workgroups
};


__global__ __launch_bounds__(GNT, 4) void route_wgrad16(WJobs js) {
  HIP_DYNAMIC_SHARED(uint16_t, glds)
  const int logical = xcd_logical(blockIdx.x, js.n);
  int t = logical % js.tiles;
  const int h = (logical / js.tiles) % js.heads, span_idx = logical / (js.tiles * js.heads);
  const bool in0 = t < js.j0.tiles;
  t -= in0 ? 0 : js.j0.tiles;
  const bool in1 = !in0 && t < js.j1.tiles;
  t -= (in0 || in1) ? 0 : js.j1.tiles;
  const bool in2 = !in0 && !in1 && t < js.j2.tiles;
  t -= (in0 || in1 || in2) ? 0 : js.j2.tiles;
  const WJob& J = in0 ? js.j0 : in1 ? js.j1 : in2 ? js.j2 : js.j3;
  const int i0 = GT * (t / J.tj), j0 = GT * (t % J.tj);
  const int rbeg = span_idx * js.span, rend = rbeg + js.span < js.R ? rbeg + js.span : js.R;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // staging role: 8x8 block (row block rb, column block cb) of A or B; the
  // operand is chosen per wave and held in scalar registers
  const bool isb = wave >= 2;
  const TnOperand O = isb ? J.b : J.a;
  const int rb = 8 * (tid & 7), cb = 8 * ((tid & 127) >> 3);
  const int col = (isb ? j0 : i0) + cb;
  const bool col_ok = col < O.width;
  const uint16_t* src = reinterpret_cast<const uint16_t*>(O.ptr) + (int64_t)h * O.hs + (col_ok ? col : 0);
  uint16_t* const stage = glds + (isb ? GT * GP : 0) + cb * GP + rb;

  // Loads are unconditional (clamped to a valid row and column) so that all
  // eight are in flight together; rows out of range are zeroed at the store.
  uint4 x[8];
  unsigned live = 0;
  auto load = [&](int k0) {
    live = 0;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int r = k0 + rb + s;
      x[s] = *reinterpret_cast<const uint4*>(src + (int64_t)(r < rend ? r : rend - 1) * O.rs);
      live |= (col_ok && r < rend) ? 1u << s : 0u;
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int s = 0; s < 8; ++s)
      if (!((live >> s) & 1)) x[s] = make_uint4(0, 0, 0, 0);
    uint16_t* const dst = stage;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const unsigned r0 = (&x[0].x)[d], r1 = (&x[1].x)[d], r2 = (&x[2].x)[d], r3 = (&x[3].x)[d];
      const unsigned r4 = (&x[4].x)[d], r5 = (&x[5].x)[d], r6 = (&x[6].x)[d], r7 = (&x[7].x)[d];
      const uint4 even = make_uint4((r0 & 0xffffu) | (r1 << 16), (r2 & 0xffffu) | (r3 << 16),
                                    (r4 & 0xffffu) | (r5 << 16), (r6 & 0xffffu) | (r7 << 16));
      const uint4 odd = make_uint4((r0 >> 16) | (r1 & 0xffff0000u), (r2 >> 16) | (r3 & 0xffff0000u),
                                   (r4 >> 16) | (r5 & 0xffff0000u), (r6 >> 16) | (r7 & 0xffff0000u));
      *reinterpret_cast<uint4*>(dst + (2 * d) * GP) = even;
      *reinterpret_cast<uint4*>(dst + (2 * d + 1) * GP) = odd;
    }
  };

  // compute role: a 64x64 quadrant of C per wave, 2x2 MFMA tiles
  const int wi = 64 * (wave & 1), wj = 64 * (wave >> 1);
  const int fr = lane & 31, fk = 8 * (lane >> 5);
  f32x16 acc[2][2] = {};

  // One LDS slab (four workgroups fit a CU); the next slab's loads are in
  // flight while this one is multiplied.
  load(rbeg);
  for (int k0 = rbeg; k0 < rend; k0 += GK) {
    store();
    __syncthreads();
    if (k0 + GK < rend) load(k0 + GK);
    const uint16_t* As = glds;
    const uint16_t* Bs = As + GT * GP;
#pragma unroll
    for (int kk = 0; kk < GK; kk += 16) {
      bf16x8 af[2], bfr[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        af[u] = *reinterpret_cast<const bf16x8*>(As + (wi + 32 * u + fr) * GP + kk + fk);
        bfr[u] = *reinterpret_cast<const bf16x8*>(Bs + (wj + 32 * u + fr) * GP + kk + fk);
      }
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int v = 0; v < 2; ++v)
          acc[u][v] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[u], bfr[v], acc[u][v], 0, 0, 0);
    }
    __syncthreads();
  }
  float* c = J.c + (int64_t)h * J.a.width * J.b.width;
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int v = 0; v < 2; ++v)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = i0 + wi + 32 * u + acc_row(r, lane >> 5), j = j0 + wj + 32 * v + fr;
        if (i < J.a.width && j < J.b.width) atomicAdd(&c[(int64_t)i * J.b.width + j], acc[u][v][r]);
      }
}

struct FourBufs {
  float* c[4];
  int64_t n[4];
};
template <bool ROUND>
__global__ void fill_or_round4(FourBufs b) {
  const int64_t step = (int64_t)gridDim.x * blockDim.x, first = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    for (int64_t i = first; i < b.n[q]; i += step) b.c[q][i] = ROUND ? round_as<bf16_t>(b.c[q][i]) : 0.f;
}

// 16-byte loads need 8-element aligned columns, strides and base.
bool wgrad16_ok(const TnOperand& o) {
  return o.width % 8 == 0 && o.rs % 8 == 0 && o.hs % 8 == 0 && (reinterpret_cast<uintptr_t>(o.ptr) & 15) == 0;
}

int check_route(const gpa_route_problem* p) {
  if (!p) return fail(GPA_HIP_EINVAL, "route: null problem");
  if (p->batch < 1 || p->tokens < 1 || p->heads < 1) return fail(GPA_HIP_EINVAL, "route: empty shape");
  if (p->slots < 1 || p->slots > RMAX || p->key_dim < 1 || p->key_dim > RMAX)
    return fail(GPA_HIP_EUNSUPPORTED, "route: slots and key width must be in [1, 256]");
  if (p->incoming < 0 || p->incoming > GPA_ROUTE_MAX_INCOMING)
    return fail(GPA_HIP_EUNSUPPORTED, "route: at most 3 incoming edges");
  if (p->dtype != GPA_DTYPE_F32 && p->dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "route: dtype");
  if ((int64_t)p->batch * p->tokens > 0x7fffffff / 2 / GPA_ROUTE_MAX_WIDTH)
    return fail(GPA_HIP_EUNSUPPORTED, "route: too many rows");
  if (!p->base.ptr || !p->q.ptr || !p->gain || !p->mlp_gain || (p->incoming && !p->edge_weight))
    return fail(GPA_HIP_EINVAL, "route: null input");
  for (int e = 0; e < p->incoming; ++e)
    if (!p->msg[e].ptr) return fail(GPA_HIP_EINVAL, "route: null message");
  if (!p->r0 || !p->h1 || !p->hd) return fail(GPA_HIP_EINVAL, "route: null saved rows");
  if (p->balanced && (!p->mix || !p->qr || !p->qdir))
    return fail(GPA_HIP_EINVAL, "route: balanced needs mix and the qr / qdir rows");
  return GPA_HIP_OK;
}

// The stride between consecutive rows r = b*T + t of a [B,T,H,X] operand, if
// rows are uniformly strided.
bool row_stride(const gpa_operand& o, int batch, int tokens, int64_t& rs) {
  if (tokens == 1) rs = o.sb;
  else if (batch == 1 || o.sb == (int64_t)tokens * o.st) rs = o.st;
  else return false;
  return true;
}

size_t fwd_lds(const gpa_route_problem& p) {
  const int kM = pad16(p.slots), k2M = pad16(2 * p.slots), kD = pad16(p.key_dim);
  return sizeof(float) * RR * ((kM + 4) + (k2M > kD ? k2M : kD) + 4);
}
size_t bwd_lds(const gpa_route_problem& p) {
  const int kM = pad16(p.slots), k2M = pad16(2 * p.slots);
  return sizeof(float) * RR * (2 * (kM + 4) + k2M + 4);
}

template <typename K>
int set_lds(K kernel, size_t bytes) {
  if (bytes > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)bytes) != hipSuccess)
    return fail(GPA_HIP_EHIP, "route: cannot raise the LDS limit");
  return GPA_HIP_OK;
}

}  // namespace
}  // namespace gpa

namespace gpa {
namespace {
// Rows read and written as 16-byte vectors: element strides multiples of 8
// (4 for float32 rows, whose 8-column pieces are two 16-byte halves).
bool vec_rows(const gpa_operand& o, int align_elems) {
  return reinterpret_cast<uintptr_t>(o.ptr) % 16 == 0 && o.sb % align_elems == 0 && o.st % align_elems == 0 &&
         o.sh % align_elems == 0;
}
bool route_vec(const gpa_route_problem& p) {
  if (p.slots % 8 || p.key_dim % 8 || !vec_rows(p.base, 4) || !vec_rows(p.q, 8)) return false;
  for (int e = 0; e < p.incoming; ++e)
    if (!vec_rows(p.msg[e], 8)) return false;
  return true;
}
bool route_bwd_vec(const gpa_route_problem& p, const gpa_route_grads& g) {
  if (!route_vec(p) || !vec_rows(g.dqo, 8) || !vec_rows(g.dbase, 4)) return false;
  if (p.balanced && (!vec_rows(g.dqr, 8) || !vec_rows(g.ddir, 8))) return false;
  for (int e = 0; e < p.incoming; ++e)
    if (!vec_rows(g.dmsg[e], 8)) return false;
  return true;
}
}  // namespace
}  // namespace gpa

namespace gpa {
namespace {
template <int BN, bool GELU, bool DUAL, typename Epi>
void launch_gemm16(const Prod& a, const Prod& b, const GemmShape& sh, const Epi& epi, hipStream_t stream) {
  const int n = sh.H * (sh.N / BN) * ((sh.R + GM_BM - 1) / GM_BM);
  hipLaunchKernelGGL((route_gemm16<BN, GELU, DUAL, Epi>), dim3(n), dim3(GM_NT), 0, stream, a, b, sh, epi);
}

// The tiled bf16 path: widths multiples of 64, 16-byte rows, the q, route and
// qo rows uniformly strided (their row strides in rs_*), and enough rows per
// head to fill 128-row tiles (a few rows, as in one-token decode, stay on the
// one-kernel path).
constexpr int TILED_MIN_ROWS = 1024;
bool route_tiled(const gpa_route_problem& p, int64_t& rs_q, int64_t& rs_route, int64_t& rs_qo) {
  return p.dtype == GPA_DTYPE_BF16 && p.slots % 64 == 0 && p.key_dim % 64 == 0 &&
         p.batch * p.tokens >= TILED_MIN_ROWS && route_vec(p) &&
         vec_rows(p.route, 8) && vec_rows(p.qo, 8) && row_stride(p.q, p.batch, p.tokens, rs_q) &&
         row_stride(p.route, p.batch, p.tokens, rs_route) && row_stride(p.qo, p.batch, p.tokens, rs_qo);
}

int route_forward_tiled(const gpa_route_problem& p, int64_t rs_q, int64_t rs_route, int64_t rs_qo,
                        hipStream_t stream) {
  const int M = p.slots, Dk = p.key_dim, R = p.batch * p.tokens, H = p.heads;
  const int64_t R64 = R;
  hipLaunchKernelGGL(route_rows16, dim3((R + RR - 1) / RR, H), dim3(RNT), 0, stream, p);
  const bf16_t* r0 = static_cast<const bf16_t*>(p.r0);
  bf16_t* h1 = static_cast<bf16_t*>(p.h1);
  bf16_t* hd = static_cast<bf16_t*>(p.hd);
  bf16_t* route = static_cast<bf16_t*>(p.route.ptr);
  // h1 = r0 U
  const Prod up{RowOp{r0, R64 * M, M}, static_cast<const bf16_t*>(p.up_t), pad32(2 * M), pad16(M), M};
  launch_gemm16<128, false, false>(up, up, GemmShape{R, 2 * M, H}, EpiH1{h1, R64 * 2 * M, 2 * M}, stream);
  // hd = gelu(h1) D, r1 = r0 + mlp_gain hd
  const Prod down{RowOp{h1, R64 * 2 * M, 2 * M}, static_cast<const bf16_t*>(p.down_t), pad32(M), pad16(2 * M),
                  2 * M};
  const EpiHd ehd{hd, r0, R64 * M, M, p.mlp_gain, route, p.route.sh, rs_route};
  // qo = r1 W_rs + query_scale q W_qs
  const Prod rs{RowOp{route, p.route.sh, rs_route}, static_cast<const bf16_t*>(p.rs_t), pad32(M), pad16(M), M};
  const Prod qs{RowOp{static_cast<const bf16_t*>(p.q.ptr), p.q.sh, rs_q}, static_cast<const bf16_t*>(p.qs_t),
                pad32(M), pad16(Dk), Dk};
  const EpiQo eqo{static_cast<bf16_t*>(p.qo.ptr), p.qo.sh, rs_qo, p.query_scale};
  const dim3 rgrid((R + RR - 1) / RR, H);
  if (M % 128 == 0) launch_gemm16<128, true, false>(down, down, GemmShape{R, M, H}, ehd, stream);
  else launch_gemm16<64, true, false>(down, down, GemmShape{R, M, H}, ehd, stream);
  // rsa_update: the route rows rescaled in place before the query product reads them
  if (p.rsa) hipLaunchKernelGGL(route_rsa_fwd<bf16_t>, rgrid, dim3(RNT), 0, stream, p);
  if (p.balanced) {
    const EpiQr eqr{static_cast<bf16_t*>(p.qr), R64 * M, M};
    const EpiQdir eqd{static_cast<bf16_t*>(p.qdir), R64 * M, M, p.query_scale};
    if (M % 128 == 0) {
      launch_gemm16<128, false, false>(rs, rs, GemmShape{R, M, H}, eqr, stream);
      launch_gemm16<128, false, false>(qs, qs, GemmShape{R, M, H}, eqd, stream);
    } else {
      launch_gemm16<64, false, false>(rs, rs, GemmShape{R, M, H}, eqr, stream);
      launch_gemm16<64, false, false>(qs, qs, GemmShape{R, M, H}, eqd, stream);
    }
    hipLaunchKernelGGL(route_mix_fwd<bf16_t>, rgrid, dim3(RNT), 0, stream, p);
  } else if (M % 128 == 0) {
    launch_gemm16<128, false, true>(rs, qs, GemmShape{R, M, H}, eqo, stream);
  } else {
    launch_gemm16<64, false, true>(rs, qs, GemmShape{R, M, H}, eqo, stream);
  }
  return check_launch("gpa_route_forward");
}
}  // namespace
}  // namespace gpa

namespace gpa {
namespace {
bool same_rows(const gpa_operand& a, const gpa_operand& b) { return a.sb == b.sb && a.st == b.st && a.sh == b.sh; }

int route_backward_tiled(const gpa_route_problem& p, const gpa_route_grads& g, int64_t rs_dqo, int64_t rs_db,
                         hipStream_t stream) {
  const int M = p.slots, Dk = p.key_dim, R = p.batch * p.tokens, H = p.heads;
  const int64_t R64 = R;
  const bf16_t* dqo = static_cast<const bf16_t*>(g.dqo.ptr);
  bf16_t* dhd = static_cast<bf16_t*>(g.dhd);
  bf16_t* dqs = static_cast<bf16_t*>(g.dqs);
  bf16_t* dh1 = static_cast<bf16_t*>(g.dh1);
  float* dr = static_cast<float*>(g.dbase.ptr);
  const dim3 rgrid((R + RR - 1) / RR, H);
  // balanced_bridge: the gradients of qr and qdir (rows [H][R][M]) and d mix first
  if (p.balanced) hipLaunchKernelGGL(route_mix_bwd<bf16_t>, rgrid, dim3(RNT), 0, stream, p, g);
  const bf16_t* d_rs = p.balanced ? static_cast<const bf16_t*>(g.dqr.ptr) : dqo;
  const bf16_t* d_qs = p.balanced ? static_cast<const bf16_t*>(g.ddir.ptr) : dqo;
  const int64_t d_sh = p.balanced ? R64 * M : g.dqo.sh, d_sr = p.balanced ? M : rs_dqo;
  // d r1 (into d base), d hd, round(query_scale dqo), d mlp_gain partials: BN = N = M
  const Prod prs{RowOp{d_rs, d_sh, d_sr}, static_cast<const bf16_t*>(p.rs), pad32(M), pad16(M), M};
  const EpiDr1 e1{d_qs, static_cast<const bf16_t*>(g.droute.ptr), g.droute.sh, rs_dqo, d_sh, d_sr, p.rsa,
                  static_cast<const bf16_t*>(p.hd), dhd, dqs, R64 * M, M, dr, g.dbase.sh, rs_db,
                  p.mlp_gain, p.query_scale, g.partials, H, 2 + p.incoming};
  const GemmShape sm{R, M, H};
  if (M == 64) launch_gemm16<64, false, false>(prs, prs, sm, e1, stream);
  else if (M == 128) launch_gemm16<128, false, false>(prs, prs, sm, e1, stream);
  else launch_gemm16<256, false, false>(prs, prs, sm, e1, stream);
  // rsa_update: d r1, d hd and the d mlp_gain partials from d r1'
  if (p.rsa) hipLaunchKernelGGL(route_rsa_bwd<bf16_t>, rgrid, dim3(RNT), 0, stream, p, g);
  // d h1 = (d hd D^T) gelu'(h1), and round(gelu(h1))
  const Prod pdown{RowOp{dhd, R64 * M, M}, static_cast<const bf16_t*>(p.down), pad32(2 * M), pad16(M), M};
  const EpiDh1 e3{static_cast<const bf16_t*>(p.h1), dh1, static_cast<bf16_t*>(g.hg), R64 * 2 * M, 2 * M};
  launch_gemm16<128, false, false>(pdown, pdown, GemmShape{R, 2 * M, H}, e3, stream);
  // d r0 = d r1 + d h1 U^T (in place), d q = round(query_scale dqo) W_qs^T
  const Prod pup{RowOp{dh1, R64 * 2 * M, 2 * M}, static_cast<const bf16_t*>(p.up), pad32(M), pad16(2 * M), 2 * M};
  const EpiDr0 e4{dr, g.dbase.sh, rs_db};
  const Prod pqs{RowOp{dqs, R64 * M, M}, static_cast<const bf16_t*>(p.qs), pad32(Dk), pad16(M), M};
  int64_t rs_dq;
  row_stride(g.dq, p.batch, p.tokens, rs_dq);
  const EpiDq e5{static_cast<bf16_t*>(g.dq.ptr), g.dq.sh, rs_dq};
  if (M % 128 == 0) launch_gemm16<128, false, false>(pup, pup, sm, e4, stream);
  else launch_gemm16<64, false, false>(pup, pup, sm, e4, stream);
  if (Dk % 128 == 0) launch_gemm16<128, false, false>(pqs, pqs, GemmShape{R, Dk, H}, e5, stream);
  else launch_gemm16<64, false, false>(pqs, pqs, GemmShape{R, Dk, H}, e5, stream);
  // softmax and relation-read backward of every row
  hipLaunchKernelGGL(route_rows16_bwd, dim3((R + RR - 1) / RR, H), dim3(RNT), 0, stream, p, g);
  return check_launch("gpa_route_backward");
}
}  // namespace
}  // namespace gpa

extern "C" int gpa_route_forward(const gpa_route_problem* problem, hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_route(problem)) return rc;
  if (!problem->up_t || !problem->down_t || !problem->rs_t || !problem->qs_t || !problem->qo.ptr ||
      !problem->route.ptr)
    return fail(GPA_HIP_EINVAL, "route: null forward weight or output");
  int64_t rs_q, rs_route, rs_qo;
  if (route_tiled(*problem, rs_q, rs_route, rs_qo)) return route_forward_tiled(*problem, rs_q, rs_route, rs_qo, stream);
  const int R = problem->batch * problem->tokens;
  const dim3 grid((R + RR - 1) / RR, problem->heads), block(RNT);
  const size_t lds = fwd_lds(*problem);
  if (problem->dtype == GPA_DTYPE_BF16 && route_vec(*problem)) {
    if (int rc = set_lds(route_fwd<bf16_t, true>, lds)) return rc;
    hipLaunchKernelGGL((route_fwd<bf16_t, true>), grid, block, lds, stream, *problem);
  } else if (problem->dtype == GPA_DTYPE_BF16) {
    if (int rc = set_lds(route_fwd<bf16_t, false>, lds)) return rc;
    hipLaunchKernelGGL((route_fwd<bf16_t, false>), grid, block, lds, stream, *problem);
  } else {
    if (int rc = set_lds(route_fwd<float, false>, lds)) return rc;
    hipLaunchKernelGGL((route_fwd<float, false>), grid, block, lds, stream, *problem);
  }
  if (problem->balanced) {
    if (problem->dtype == GPA_DTYPE_BF16)
      hipLaunchKernelGGL(route_mix_fwd<bf16_t>, grid, block, 0, stream, *problem);
    else
      hipLaunchKernelGGL(route_mix_fwd<float>, grid, block, 0, stream, *problem);
  }
  return check_launch("gpa_route_forward");
}

extern "C" int gpa_route_forward_many(const gpa_route_problem* problems, int32_t n, hipStream_t stream) {
  using namespace gpa;
  if (!problems || n < 1 || n > GPA_ROUTE_MAX_PACK) return fail(GPA_HIP_EINVAL, "route: 1 to 4 problems");
  bool pack = n > 1;
  for (int i = 0; i < n; ++i) {
    const gpa_route_problem& p = problems[i];
    if (int rc = check_route(&p)) return rc;
    if (!p.up_t || !p.down_t || !p.rs_t || !p.qs_t || !p.qo.ptr || !p.route.ptr)
      return fail(GPA_HIP_EINVAL, "route: null forward weight or output");
    int64_t rs_q, rs_route, rs_qo;
    // (the packed kernel is instantiated for the bf16 16-byte row path only)
    if (route_tiled(p, rs_q, rs_route, rs_qo) || p.dtype != GPA_DTYPE_BF16 || !route_vec(p)) pack = false;
  }
  if (!pack) {
    for (int i = 0; i < n; ++i)
      if (int rc = gpa_route_forward(&problems[i], stream)) return rc;
    return GPA_HIP_OK;
  }
  RoutePack pk{};
  pk.n = n;
  int total = 0;
  size_t lds = 0;
  for (int i = 0; i < n; ++i) {
    const gpa_route_problem& p = problems[i];
    pk.p[i] = p;
    pk.wg0[i] = total;
    pk.tiles[i] = (p.batch * p.tokens + RR - 1) / RR;
    total += pk.tiles[i] * p.heads;
    lds = std::max(lds, fwd_lds(p));
  }
  if (int rc = set_lds(route_fwd_pack, lds)) return rc;
  hipLaunchKernelGGL(route_fwd_pack, dim3(total), dim3(64 * RPACK_W), lds, stream, pk);
  for (int i = 0; i < n; ++i)
    if (problems[i].balanced)
      hipLaunchKernelGGL(route_mix_fwd<bf16_t>, dim3(pk.tiles[i], problems[i].heads), dim3(RNT), 0, stream,
                         problems[i]);
  return check_launch("gpa_route_forward_many");
}

extern "C" int gpa_route_backward(const gpa_route_problem* problem, const gpa_route_grads* grads,
                                  hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_route(problem)) return rc;
  if (!grads || !grads->dqo.ptr || !grads->dbase.ptr || !grads->dq.ptr || !grads->dh1 || !grads->dhd ||
      !grads->dqs || !grads->hg || !grads->partials || !problem->up || !problem->down || !problem->rs || !problem->qs)
    return fail(GPA_HIP_EINVAL, "route: null gradient buffer or backward weight");
  for (int e = 0; e < problem->incoming; ++e)
    if (!grads->dmsg[e].ptr) return fail(GPA_HIP_EINVAL, "route: null message gradient");
  if (problem->balanced && (!grads->dqr.ptr || !grads->ddir.ptr || !grads->mix_partials))
    return fail(GPA_HIP_EINVAL, "route: balanced needs the qr / qdir gradient rows and mix partials");
  {
    int64_t rs_q, rs_route, rs_qo, rs_dqo, rs_db, rs_dq;
    if (route_tiled(*problem, rs_q, rs_route, rs_qo) && route_bwd_vec(*problem, *grads) &&
        row_stride(grads->dqo, problem->batch, problem->tokens, rs_dqo) &&
        row_stride(grads->dbase, problem->batch, problem->tokens, rs_db) &&
        row_stride(grads->dq, problem->batch, problem->tokens, rs_dq) &&
        vec_rows(grads->dq, 8) && (!grads->droute.ptr || (same_rows(grads->droute, grads->dqo) &&
                                                           vec_rows(grads->droute, 8))))
      return route_backward_tiled(*problem, *grads, rs_dqo, rs_db, stream);
  }
  const int R = problem->batch * problem->tokens;
  const dim3 grid((R + RR - 1) / RR, problem->heads), block(RNT);
  const size_t lds = bwd_lds(*problem);
  if (problem->balanced) {  // the gradients of qr and qdir, which route_bwd reads
    if (problem->dtype == GPA_DTYPE_BF16)
      hipLaunchKernelGGL(route_mix_bwd<bf16_t>, grid, block, 0, stream, *problem, *grads);
    else
      hipLaunchKernelGGL(route_mix_bwd<float>, grid, block, 0, stream, *problem, *grads);
  }
  if (problem->dtype == GPA_DTYPE_BF16 && route_bwd_vec(*problem, *grads)) {
    if (int rc = set_lds(route_bwd<bf16_t, true>, lds)) return rc;
    hipLaunchKernelGGL((route_bwd<bf16_t, true>), grid, block, lds, stream, *problem, *grads);
  } else if (problem->dtype == GPA_DTYPE_BF16) {
    if (int rc = set_lds(route_bwd<bf16_t, false>, lds)) return rc;
    hipLaunchKernelGGL((route_bwd<bf16_t, false>), grid, block, lds, stream, *problem, *grads);
  } else {
    if (int rc = set_lds(route_bwd<float, false>, lds)) return rc;
    hipLaunchKernelGGL((route_bwd<float, false>), grid, block, lds, stream, *problem, *grads);
  }
  return check_launch("gpa_route_backward");
}

namespace gpa {
int launch_tn_products(const TnProduct* products, int np, int H, int R, bool bf, hipStream_t stream) {
  if (np < 1 || np > 4) return fail(GPA_HIP_EINVAL, "tn products: 1 to 4 products");
  struct Job {
    TnOperand a, b;
    float* c;
  } jobs[4];
  for (int q = 0; q < np; ++q)
    jobs[q] = {{products[q].a, products[q].a_rs, products[q].a_hs, products[q].a_width},
               {products[q].b, products[q].b_rs, products[q].b_hs, products[q].b_width},
               products[q].c};
  bool fast = bf;
  for (int q = 0; q < np; ++q) fast = fast && wgrad16_ok(jobs[q].a) && wgrad16_ok(jobs[q].b);
  if (fast) {
    WJob w[4] = {};  // unused products have no tiles
    FourBufs fb = {};
    int tiles = 0;
    for (int q = 0; q < np; ++q) {
      const int ti = (jobs[q].a.width + GT - 1) / GT, tj = (jobs[q].b.width + GT - 1) / GT;
      w[q] = {jobs[q].a, jobs[q].b, jobs[q].c, tj, ti * tj};
      fb.c[q] = jobs[q].c;
      fb.n[q] = (int64_t)H * jobs[q].a.width * jobs[q].b.width;
      tiles += ti * tj;
    }
    // Row spans: enough workgroups for the whole chip, each span whole slabs.
    const int slabs = (R + GK - 1) / GK, per_span_wgs = tiles * H;
    int spans = (G_WGS + per_span_wgs - 1) / per_span_wgs;
    spans = spans < 1 ? 1 : spans > slabs ? slabs : spans;
    const int span = GK * ((slabs + spans - 1) / spans);
    spans = (R + span - 1) / span;
    const int n = tiles * H * spans;
    const WJobs js{w[0], w[1], w[2], w[3], span, R, tiles, H, n};
    if (int rc = set_lds(route_wgrad16, G_LDS)) return rc;
    const int64_t total = fb.n[0] + fb.n[1] + fb.n[2] + fb.n[3];
    const dim3 fgrid((unsigned)((total + 1023) / 1024 < 2048 ? (total + 1023) / 1024 : 2048));
    hipLaunchKernelGGL(fill_or_round4<false>, fgrid, dim3(256), 0, stream, fb);
    hipLaunchKernelGGL(route_wgrad16, dim3(n), dim3(GNT), G_LDS, stream, js);
    hipLaunchKernelGGL(fill_or_round4<true>, fgrid, dim3(256), 0, stream, fb);
    return GPA_HIP_OK;
  }
  for (int q = 0; q < np; ++q) {
    const Job& j = jobs[q];
    const int64_t n = (int64_t)H * j.a.width * j.b.width;
    const dim3 fill_grid((unsigned)((n + 255) / 256 < 64 ? (n + 255) / 256 : 64));
    hipLaunchKernelGGL(fill_zero, fill_grid, dim3(256), 0, stream, j.c, n);
    const dim3 grid(((j.a.width + WT - 1) / WT) * ((j.b.width + WT - 1) / WT), H, (R + WKC - 1) / WKC);
    if (bf)
      hipLaunchKernelGGL(route_wgrad<bf16_t>, grid, dim3(RNT), 0, stream, j.a, j.b, j.c, R);
    else
      hipLaunchKernelGGL(route_wgrad<float>, grid, dim3(RNT), 0, stream, j.a, j.b, j.c, R);
    if (bf) hipLaunchKernelGGL(round_in_place<bf16_t>, fill_grid, dim3(256), 0, stream, j.c, n);
  }
  return GPA_HIP_OK;
}
}  // namespace gpa

extern "C" int gpa_route_weight_grads(const gpa_route_problem* problem, const gpa_route_grads* grads, float* d_up,
                                      float* d_down, float* d_rs, float* d_qs, hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_route(problem)) return rc;
  if (!grads || !grads->dqo.ptr || !grads->dh1 || !grads->dhd || !grads->dqs || !grads->hg || !problem->route.ptr || !d_up ||
      !d_down || !d_rs || !d_qs)
    return fail(GPA_HIP_EINVAL, "route: null weight-gradient buffer");
  const int M = problem->slots, Dk = problem->key_dim, R = problem->batch * problem->tokens, H = problem->heads;
  // Rows r = b*T + t of a [B,T,H,X] operand must sit at r * (row stride).
  int64_t rs_route, rs_dqo, rs_q;
  if (!row_stride(problem->route, problem->batch, problem->tokens, rs_route) ||
      !row_stride(grads->dqo, problem->batch, problem->tokens, rs_dqo) ||
      !row_stride(problem->q, problem->batch, problem->tokens, rs_q))
    return fail(GPA_HIP_EINVAL, "route: route, dqo and q rows must be uniformly strided");
  const int64_t R64 = R;
  const TnOperand r0{problem->r0, M, R64 * M, M};
  const TnOperand hid{grads->hg, 2 * M, R64 * 2 * M, 2 * M};
  const TnOperand dh1{grads->dh1, 2 * M, R64 * 2 * M, 2 * M};
  const TnOperand dhd{grads->dhd, M, R64 * M, M};
  const TnOperand dqs{grads->dqs, M, R64 * M, M};
  const TnOperand r1{problem->route.ptr, rs_route, problem->route.sh, M};
  // d W_rs = r1^T (the gradient of qr: dqo, or its balanced_bridge form)
  const TnOperand dqo = problem->balanced ? TnOperand{grads->dqr.ptr, M, R64 * M, M}
                                          : TnOperand{grads->dqo.ptr, rs_dqo, grads->dqo.sh, M};
  const TnOperand q{problem->q.ptr, rs_q, problem->q.sh, Dk};
  auto prod = [](const TnOperand& a, const TnOperand& b, float* c) {
    return TnProduct{a.ptr, a.rs, a.hs, a.width, b.ptr, b.rs, b.hs, b.width, c};
  };
  const TnProduct products[4] = {prod(r0, dh1, d_up), prod(hid, dhd, d_down), prod(r1, dqo, d_rs), prod(q, dqs, d_qs)};
  if (int rc = launch_tn_products(products, 4, H, R, problem->dtype == GPA_DTYPE_BF16, stream)) return rc;
  return check_launch("gpa_route_weight_grads");
}
