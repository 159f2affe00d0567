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

template <typename E, bool VEC>
__global__ __launch_bounds__(RNT) void route_fwd(gpa_route_problem p) {
  using W = typename Wt<E>::type;
  HIP_DYNAMIC_SHARED(float, lds)
  const int M = p.slots, Dk = p.key_dim, R = p.batch * p.tokens;
  const RouteTile rtile = route_tile();
  const int h = rtile.h, row0 = rtile.tile * RR;
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
  if constexpr (VEC) {
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
      if (c < kM) {
        *reinterpret_cast<f32x4*>(&A[row * lda + c]) = f32x4{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<f32x4*>(&A[row * lda + c + 4]) = f32x4{v[4], v[5], v[6], v[7]};
      }
      if (valid && on) *reinterpret_cast<uint4*>(sr0 + (int64_t)r * M + c) = pack_bf8(v);
    }
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
    for (int t = wave; t < pad32(2 * M) / 32; t += RW) {
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
    for (int t = wave; t < pad32(M) / 32; t += RW) {
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
            route[rows.at(p.route, r, h) + col] = from_f32<E>(r1);
          }
        }
      }
    }
  }
  __syncthreads();

  // ---- q -> Hs
  if constexpr (VEC) {
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
    for (int t = wave; t < pad32(M) / 32; t += RW) {
      f32x16 a3 = {}, a4 = {};
      tile_gemm(a3, A, lda, rt, kM, kM, 32 * t, lane);
      tile_gemm(a4, Hs, ldh, qt, kD, kD, 32 * t, lane);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = acc_row(i, lane >> 5), col = 32 * t + (lane & 31), r = row0 + row;
        if (col < M && r < R) {
          const float dir = round_as<E>(p.query_scale * round_as<E>(a4[i]));
          qo[rows.at(p.qo, r, h) + col] = from_f32<E>(round_as<E>(round_as<E>(a3[i]) + dir));
        }
      }
    }
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

  // ---- dqo -> G
  if constexpr (VEC) {
    const int c = 8 * (tid & 31), rsub = tid >> 5;
    uint4 dv[VPASS];
#pragma unroll
    for (int i = 0; i < VPASS; ++i) {
      const int r = row0 + rsub + 8 * i;
      dv[i] = (c < M && r < R) ? *reinterpret_cast<const uint4*>(reinterpret_cast<const bf16_t*>(g.dqo.ptr) +
                                                                  rows.at(g.dqo, r, h) + c)
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
    const E* dqo = reinterpret_cast<const E*>(g.dqo.ptr) + rows.at(g.dqo, valid ? r : R - 1, h);
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

  // ---- G <- round(query_scale dqo) (the gradient of q W_qs)
  if constexpr (VEC) {
    const int c = 8 * (tid & 31), rsub = tid >> 5;
    if (c < M) {
#pragma unroll
      for (int i = 0; i < VPASS; ++i) {
        const int row = rsub + 8 * i, r = row0 + row;
        float* gr = &G[row * lda + c];
        const f32x4 a = *reinterpret_cast<const f32x4*>(gr), b = *reinterpret_cast<const f32x4*>(gr + 4);
        float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = round_as<E>(p.query_scale * x[e]);
        *reinterpret_cast<f32x4*>(gr) = f32x4{x[0], x[1], x[2], x[3]};
        *reinterpret_cast<f32x4*>(gr + 4) = f32x4{x[4], x[5], x[6], x[7]};
        if (r < R) *reinterpret_cast<uint4*>(gdqs + (int64_t)r * M + c) = pack_bf8(x);
      }
    }
  } else {
    const int row = tid >> 3, part = tid & 7, r = row0 + row;
#pragma unroll
    for (int i = 0; i < RPER; ++i) {
      const int m = part + 8 * i;
      if (m < M) {
        const float x = round_as<E>(p.query_scale * G[row * lda + m]);
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
      float d0[8] = {};
      if (on) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(&A2[row * lda + c]);
        const f32x4 b = *reinterpret_cast<const f32x4*>(&A2[row * lda + c + 4]);
        d0[0] = a.x; d0[1] = a.y; d0[2] = a.z; d0[3] = a.w; d0[4] = b.x; d0[5] = b.y; d0[6] = b.z; d0[7] = b.w;
      }
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
  for (int e = 0; e < p.incoming; ++e)
    if (!vec_rows(g.dmsg[e], 8)) return false;
  return true;
}
}  // namespace
}  // namespace gpa

extern "C" int gpa_route_forward(const gpa_route_problem* problem, hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_route(problem)) return rc;
  if (!problem->up_t || !problem->down_t || !problem->rs_t || !problem->qs_t || !problem->qo.ptr ||
      !problem->route.ptr)
    return fail(GPA_HIP_EINVAL, "route: null forward weight or output");
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
  return check_launch("gpa_route_forward");
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
  const int R = problem->batch * problem->tokens;
  const dim3 grid((R + RR - 1) / RR, problem->heads), block(RNT);
  const size_t lds = bwd_lds(*problem);
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
  const TnOperand dqo{grads->dqo.ptr, rs_dqo, grads->dqo.sh, M};
  const TnOperand q{problem->q.ptr, rs_q, problem->q.sh, Dk};
  auto prod = [](const TnOperand& a, const TnOperand& b, float* c) {
    return TnProduct{a.ptr, a.rs, a.hs, a.width, b.ptr, b.rs, b.hs, b.width, c};
  };
  const TnProduct products[4] = {prod(r0, dh1, d_up), prod(hid, dhd, d_down), prod(r1, dqo, d_rs), prod(q, dqs, d_qs)};
  if (int rc = launch_tn_products(products, 4, H, R, problem->dtype == GPA_DTYPE_BF16, stream)) return rc;
  return check_launch("gpa_route_weight_grads");
}
