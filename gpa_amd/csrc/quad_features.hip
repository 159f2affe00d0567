// Quadratic Q/K feature map (reference src/gpa/features.py:17-25), forward and
// backward, one workgroup per (32-row tile, head):
//   u = unit(x) rounded to E;  a = u L, b = u R (E products, float32 accumulation,
//   rounded to E);  z = u + (c a) b with c = 2 sigmoid(gain_raw) sqrt(D);
//   out = unit(z) ||x||_eps rounded to E.
// The two products run on the MFMA (v_mfma_f32_32x32x16_bf16 for bf16,
// v_mfma_f32_32x32x2f32 for float32) with u staged in LDS and the weights read
// as 16-byte rows of a transposed, zero-padded copy (the caller prepares it:
// the weights are parameters, a few hundred KB).  Wave w owns the column
// blocks w, w + 4 of both products, so a and b of an element meet in one
// lane's accumulators; row sums go through half-wave shuffles and LDS.
//
// The backward recomputes the forward, forms dz through the two
// normalisations, da = (dz b) c and db = dz (c a) rounded to E, and
// du = dz + da L^T + db R^T as one MFMA product over the concatenated
// [da | db] rows; dx follows through unit(x) and ||x||.  It also writes u and
// [da | db] head-major for the weight gradients u^T [da | db] (a plain
// batched GEMM the caller runs) and one partial sum of dc per workgroup.
#include <hip/hip_runtime.h>

#include "mfma_tiles.h"

namespace gpa {
namespace {

constexpr int QT = 256;   // threads per workgroup (4 waves)
constexpr int QR = 32;    // rows per workgroup
constexpr int QMAXB = 2;  // column blocks per wave (dim <= 256)

__host__ __device__ inline int qpad(int d) { return (d + 31) / 32 * 32; }
__device__ __forceinline__ int qmin(int a, int b) { return a < b ? a : b; }

template <typename E>
struct QLayout {
  int DP, NB, ULD, DLD;
  E* u;        // [32][ULD]  unit(x) rows
  E* dab;      // [32][DLD]  d(a) | d(b) rows (backward)
  float* nrm;  // [32] ||x||_eps = sqrt(sum x^2 + 1e-12)
  float* xn;   // [32] sqrt(sum x^2)
  float* part; // [3][8][32] per-block row partial sums
  float* row;  // [3][32] row totals
  float* wsum; // [4] per-wave partial of dc
};

template <typename E>
__host__ __device__ inline size_t q_lds_bytes(int dim, bool backward) {
  const int DP = qpad(dim), ULD = DP + 16 / (int)sizeof(E), DLD = 2 * DP + 16 / (int)sizeof(E);
  size_t b = (size_t)QR * ULD * sizeof(E) + (backward ? (size_t)QR * DLD * sizeof(E) : 0);
  return b + (2 * QR + 3 * 8 * QR + 3 * QR + 4) * sizeof(float);
}

template <typename E>
__device__ QLayout<E> q_layout(char* smem, int dim, bool backward) {
  QLayout<E> L;
  L.DP = qpad(dim);
  L.NB = L.DP / 32;
  L.ULD = L.DP + 16 / (int)sizeof(E);
  L.DLD = 2 * L.DP + 16 / (int)sizeof(E);
  char* p = smem;
  L.u = reinterpret_cast<E*>(p);
  p += (size_t)QR * L.ULD * sizeof(E);
  L.dab = reinterpret_cast<E*>(p);
  if (backward) p += (size_t)QR * L.DLD * sizeof(E);
  float* f = reinterpret_cast<float*>(p);
  L.nrm = f;
  L.xn = f + QR;
  L.part = f + 2 * QR;
  L.row = L.part + 3 * 8 * QR;
  L.wsum = L.row + 3 * QR;
  return L;
}

// Rows r0 .. r0+31 of head h: u into LDS (zero past dim and past the last row),
// ||x|| and ||x||_eps per row.
template <typename E>
__device__ void q_rows(const gpa_quad_problem& p, int h, int r0, QLayout<E>& L) {
  const int tid = threadIdx.x, row = tid / 8, part = tid % 8, D = p.dim;
  const int grow = qmin(r0 + row, p.rows - 1);
  const E* xr = reinterpret_cast<const E*>(p.x) + (int64_t)grow * p.row_stride + (int64_t)h * D;
  float xv[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) xv[i] = to_f32(xr[qmin(part + 8 * i, D - 1)]);
  const bool live = r0 + row < p.rows;
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    xv[i] = (live && part + 8 * i < D) ? xv[i] : 0.f;
    ss += xv[i] * xv[i];
  }
  ss += __shfl_xor(ss, 1, 64);
  ss += __shfl_xor(ss, 2, 64);
  ss += __shfl_xor(ss, 4, 64);
  const float n = sqrtf(ss), den = fmaxf(n, 1e-6f);
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const int d = part + 8 * i;
    if (d < L.DP) L.u[row * L.ULD + d] = from_f32<E>(xv[i] / den);
  }
  if (part == 0) {
    L.nrm[row] = sqrtf(ss + 1e-12f);
    L.xn[row] = n;
  }
}

// acc_a, acc_b = u W_p for the 32 columns of block cb (p = 0: left, 1: right).
template <typename E>
__device__ __forceinline__ void q_products(const gpa_quad_problem& p, int h, int cb, const QLayout<E>& L,
                                           f32x16& acc_a, f32x16& acc_b) {
  const int l = threadIdx.x & 63, lr = l & 31, hi = l >> 5;
  const E* wt = reinterpret_cast<const E*>(p.wt);
  const E* wl = wt + ((int64_t)(h * 2 + 0) * L.DP + cb * 32 + lr) * L.DP;
  const E* wr = wt + ((int64_t)(h * 2 + 1) * L.DP + cb * 32 + lr) * L.DP;
  for (int i = 0; i < 16; ++i) acc_a[i] = acc_b[i] = 0.f;
  if constexpr (sizeof(E) == 2) {
    const bf16_t* u = reinterpret_cast<const bf16_t*>(L.u);
    for (int ks = 0; ks < L.DP / 16; ++ks) {
      const int k0 = 16 * ks + 8 * hi;
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(u + lr * L.ULD + k0);
      const bf16x8 bl = *reinterpret_cast<const bf16x8*>(wl + k0);
      const bf16x8 br = *reinterpret_cast<const bf16x8*>(wr + k0);
      mma_bf16(acc_a, a, bl);
      mma_bf16(acc_b, a, br);
    }
  } else {
    const float* u = reinterpret_cast<const float*>(L.u);
    for (int ks = 0; ks < L.DP / 8; ++ks) {
      const int c0 = 8 * ks + 4 * hi;
      const f32x4 a = ld_c(u, L.ULD, lr, c0);
      const f32x4 bl = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(wl) + c0);
      const f32x4 br = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(wr) + c0);
      mma8(acc_a, a, bl);
      mma8(acc_b, a, br);
    }
  }
}

// Row sums of a lane's 16 accumulator-layout values over the block's 32
// columns, into part[slot][cb][row].
__device__ __forceinline__ void q_row_part(float (&v)[16], float* part, int slot, int cb) {
  const int l = threadIdx.x & 63;
  const float s = tile_row_sum(v, l);
  if ((l & 1) == 0) part[(slot * 8 + cb) * QR + acc_row(sum_index(l), l >> 5)] = s;
}

// row[slot][r] = sum over the column blocks of part[slot][.][r] (threads 0..31).
__device__ __forceinline__ void q_row_total(float* part, float* row, int slot, int nb) {
  const int t = threadIdx.x;
  if (t < QR) {
    float s = 0.f;
    for (int cb = 0; cb < nb; ++cb) s += part[(slot * 8 + cb) * QR + t];
    row[slot * QR + t] = s;
  }
}

template <typename E>
__global__ __launch_bounds__(QT) void quad_fwd(gpa_quad_problem p) {
  HIP_DYNAMIC_SHARED(char, smem)
  const int h = blockIdx.y, r0 = blockIdx.x * QR, w = threadIdx.x >> 6, l = threadIdx.x & 63;
  QLayout<E> L = q_layout<E>(smem, p.dim, false);
  q_rows<E>(p, h, r0, L);
  __syncthreads();
  const float c = p.gain[h];
  float z[QMAXB][16];
#pragma unroll
  for (int bi = 0; bi < QMAXB; ++bi) {
    const int cb = w + 4 * bi;
    if (cb >= L.NB) break;
    f32x16 acc_a, acc_b;
    q_products<E>(p, h, cb, L, acc_a, acc_b);
    float zz[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = acc_row(r, l >> 5), col = cb * 32 + (l & 31);
      const float a = round_as<E>(acc_a[r]), b = round_as<E>(acc_b[r]);
      z[bi][r] = to_f32(L.u[row * L.ULD + col]) + (c * a) * b;
      zz[r] = z[bi][r] * z[bi][r];
    }
    q_row_part(zz, L.part, 0, cb);
  }
  __syncthreads();
  q_row_total(L.part, L.row, 0, L.NB);
  __syncthreads();
  E* out = reinterpret_cast<E*>(p.out);
#pragma unroll
  for (int bi = 0; bi < QMAXB; ++bi) {
    const int cb = w + 4 * bi;
    if (cb >= L.NB) break;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = acc_row(r, l >> 5), col = cb * 32 + (l & 31);
      const float zn = fmaxf(sqrtf(L.row[row]), 1e-6f);
      if (r0 + row < p.rows && col < p.dim)
        out[((int64_t)(r0 + row) * p.heads + h) * p.dim + col] = from_f32<E>(z[bi][r] / zn * L.nrm[row]);
    }
  }
}

template <typename E>
__global__ __launch_bounds__(QT) void quad_bwd(gpa_quad_problem p, gpa_quad_grads g) {
  HIP_DYNAMIC_SHARED(char, smem)
  const int h = blockIdx.y, r0 = blockIdx.x * QR, w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int D = p.dim;
  QLayout<E> L = q_layout<E>(smem, D, true);
  q_rows<E>(p, h, r0, L);
  __syncthreads();
  const float c = p.gain[h];
  float z[QMAXB][16], av[QMAXB][16], bv[QMAXB][16];
#pragma unroll
  for (int bi = 0; bi < QMAXB; ++bi) {
    const int cb = w + 4 * bi;
    if (cb >= L.NB) break;
    f32x16 acc_a, acc_b;
    q_products<E>(p, h, cb, L, acc_a, acc_b);
    float zz[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = acc_row(r, l >> 5), col = cb * 32 + (l & 31);
      av[bi][r] = round_as<E>(acc_a[r]);
      bv[bi][r] = round_as<E>(acc_b[r]);
      z[bi][r] = to_f32(L.u[row * L.ULD + col]) + (c * av[bi][r]) * bv[bi][r];
      zz[r] = z[bi][r] * z[bi][r];
    }
    q_row_part(zz, L.part, 0, cb);
  }
  __syncthreads();
  q_row_total(L.part, L.row, 0, L.NB);
  __syncthreads();
  // out = unit(z) nrm: d nrm = sum g unit(z), d unit(z) = g nrm; the
  // normalisation backward needs sum d unit(z) . z per row.
  const E* dout = reinterpret_cast<const E*>(g.dout);
  float gv[QMAXB][16];
#pragma unroll
  for (int bi = 0; bi < QMAXB; ++bi) {
    const int cb = w + 4 * bi;
    if (cb >= L.NB) break;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = acc_row(r, l >> 5), col = cb * 32 + (l & 31);
      gv[bi][r] = to_f32(dout[((int64_t)qmin(r0 + row, p.rows - 1) * p.heads + h) * D + qmin(col, D - 1)]);
    }
    float s1[16], s2[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = acc_row(r, l >> 5), col = cb * 32 + (l & 31);
      if (!(r0 + row < p.rows && col < D)) gv[bi][r] = 0.f;
      const float zn = fmaxf(sqrtf(L.row[row]), 1e-6f);
      s1[r] = gv[bi][r] * (z[bi][r] / zn);
      s2[r] = gv[bi][r] * L.nrm[row] * z[bi][r];
    }
    q_row_part(s1, L.part, 1, cb);
    q_row_part(s2, L.part, 2, cb);
  }
  __syncthreads();
  q_row_total(L.part, L.row, 1, L.NB);
  q_row_total(L.part, L.row, 2, L.NB);
  __syncthreads();
  // dz, then da = (dz b) c, db = dz (c a) in E; du starts as dz rounded to E.
  float du0[QMAXB][16];
  float dc = 0.f;
  E* uo = reinterpret_cast<E*>(g.u);
  E* dabo = reinterpret_cast<E*>(g.dab);
#pragma unroll
  for (int bi = 0; bi < QMAXB; ++bi) {
    const int cb = w + 4 * bi;
    if (cb >= L.NB) break;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = acc_row(r, l >> 5), col = cb * 32 + (l & 31);
      const float zt = sqrtf(L.row[row]);
      const float du = gv[bi][r] * L.nrm[row];
      float dz;
      if (zt > 1e-6f) dz = du / zt - z[bi][r] * (L.row[2 * QR + row] / (zt * zt * zt));
      else dz = du / 1e-6f;
      const float t1 = dz * bv[bi][r];
      dc += t1 * av[bi][r];
      const E da = from_f32<E>(t1 * c), db = from_f32<E>(dz * (c * av[bi][r]));
      L.dab[row * L.DLD + col] = da;
      L.dab[row * L.DLD + L.DP + col] = db;
      du0[bi][r] = round_as<E>(dz);
      if (r0 + row < p.rows) {
        const int64_t hr = (int64_t)h * p.rows + r0 + row;
        dabo[hr * 2 * L.DP + col] = da;
        dabo[hr * 2 * L.DP + L.DP + col] = db;
        uo[hr * L.DP + col] = L.u[row * L.ULD + col];
      }
    }
  }
  dc = sum64(dc);
  if (l == 0) L.wsum[w] = dc;
  __syncthreads();
  if (threadIdx.x == 0) g.dgain[(int64_t)blockIdx.x * p.heads + h] = L.wsum[0] + L.wsum[1] + L.wsum[2] + L.wsum[3];
  // du = dz + da L^T + db R^T: contraction over the 2 DP columns of [da | db];
  // the B operand of output column k is row k of w = [L | R] (contiguous).
  const E* wk = reinterpret_cast<const E*>(p.w);
  float dun[QMAXB][16];
#pragma unroll
  for (int bi = 0; bi < QMAXB; ++bi) {
    const int cb = w + 4 * bi;
    if (cb >= L.NB) break;
    f32x16 acc_l, acc_r;
    for (int i = 0; i < 16; ++i) acc_l[i] = acc_r[i] = 0.f;
    const int lr = l & 31, hi = l >> 5;
    const E* wrow = wk + ((int64_t)h * L.DP + cb * 32 + lr) * 2 * L.DP;
    if constexpr (sizeof(E) == 2) {
      const bf16_t* d = reinterpret_cast<const bf16_t*>(L.dab);
      for (int ks = 0; ks < L.DP / 16; ++ks) {
        const int k0 = 16 * ks + 8 * hi;
        mma_bf16(acc_l, *reinterpret_cast<const bf16x8*>(d + lr * L.DLD + k0),
                 *reinterpret_cast<const bf16x8*>(wrow + k0));
        mma_bf16(acc_r, *reinterpret_cast<const bf16x8*>(d + lr * L.DLD + L.DP + k0),
                 *reinterpret_cast<const bf16x8*>(wrow + L.DP + k0));
      }
    } else {
      const float* d = reinterpret_cast<const float*>(L.dab);
      const float* wf = reinterpret_cast<const float*>(wrow);
      for (int ks = 0; ks < L.DP / 8; ++ks) {
        const int c0 = 8 * ks + 4 * hi;
        mma8(acc_l, ld_c(d, L.DLD, lr, c0), *reinterpret_cast<const f32x4*>(wf + c0));
        mma8(acc_r, ld_c(d, L.DLD, lr, L.DP + c0), *reinterpret_cast<const f32x4*>(wf + L.DP + c0));
      }
    }
    // x of the same elements, for unit(x)'s backward
    const E* x = reinterpret_cast<const E*>(p.x);
    float xv[16], s3[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = acc_row(r, l >> 5), col = cb * 32 + lr;
      xv[r] = to_f32(x[(int64_t)qmin(r0 + row, p.rows - 1) * p.row_stride + (int64_t)h * D + qmin(col, D - 1)]);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = acc_row(r, l >> 5), col = cb * 32 + lr;
      if (!(r0 + row < p.rows && col < D)) xv[r] = 0.f;
      dun[bi][r] = round_as<E>(du0[bi][r] + round_as<E>(acc_l[r]) + round_as<E>(acc_r[r]));
      s3[r] = dun[bi][r] * xv[r];
      av[bi][r] = xv[r];  // keep x for dx
    }
    q_row_part(s3, L.part, 0, cb);
  }
  __syncthreads();
  q_row_total(L.part, L.row, 0, L.NB);
  __syncthreads();
  E* dx = reinterpret_cast<E*>(g.dx);
#pragma unroll
  for (int bi = 0; bi < QMAXB; ++bi) {
    const int cb = w + 4 * bi;
    if (cb >= L.NB) break;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = acc_row(r, l >> 5), col = cb * 32 + (l & 31);
      const float n = L.xn[row], x = av[bi][r];
      float d;
      if (n > 1e-6f) d = dun[bi][r] / n - x * (L.row[row] / (n * n * n));
      else d = dun[bi][r] / 1e-6f;
      d += L.row[QR + row] * x / L.nrm[row];  // through ||x||_eps
      if (r0 + row < p.rows && col < D) dx[((int64_t)(r0 + row) * p.heads + h) * D + col] = from_f32<E>(d);
    }
  }
}

int check_quad(const gpa_quad_problem* pp) {
  if (!pp) return fail(GPA_HIP_EINVAL, "quad features: null problem");
  const gpa_quad_problem& p = *pp;
  if (p.rows < 1 || p.heads < 1 || p.dim < 1 || p.dim > GPA_QUAD_MAX_DIM)
    return fail(GPA_HIP_EINVAL, "quad features: rows, heads positive, dim 1..GPA_QUAD_MAX_DIM");
  if (p.dtype != GPA_DTYPE_F32 && p.dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "quad features: dtype");
  if (!p.x || !p.wt || !p.w || !p.gain || p.row_stride < (int64_t)p.heads * p.dim)
    return fail(GPA_HIP_EINVAL, "quad features: x, wt, w, gain required; row_stride >= heads*dim");
  if ((int64_t)(p.rows + QR - 1) / QR > 0x7fffffff || p.heads > 65535)
    return fail(GPA_HIP_EINVAL, "quad features: too many rows or heads");
  return 0;
}

template <typename K>
int q_lds_attr(K kernel, size_t bytes) {
  if (bytes <= 65536) return 0;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)bytes) != hipSuccess)
    return fail(GPA_HIP_EHIP, "hipFuncSetAttribute(max dynamic LDS) failed");
  return 0;
}

}  // namespace
}  // namespace gpa

extern "C" int gpa_quad_features_forward(const gpa_quad_problem* problem, hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_quad(problem)) return rc;
  const gpa_quad_problem& p = *problem;
  if (!p.out) return fail(GPA_HIP_EINVAL, "quad features: out required");
  const dim3 grid((unsigned)((p.rows + QR - 1) / QR), (unsigned)p.heads);
  if (p.dtype == GPA_DTYPE_BF16) {
    const size_t lds = q_lds_bytes<bf16_t>(p.dim, false);
    if (int rc = q_lds_attr(quad_fwd<bf16_t>, lds)) return rc;
    hipLaunchKernelGGL((quad_fwd<bf16_t>), grid, dim3(QT), lds, stream, p);
  } else {
    const size_t lds = q_lds_bytes<float>(p.dim, false);
    if (int rc = q_lds_attr(quad_fwd<float>, lds)) return rc;
    hipLaunchKernelGGL((quad_fwd<float>), grid, dim3(QT), lds, stream, p);
  }
  return check_launch("gpa_quad_features_forward");
}

extern "C" int gpa_quad_features_backward(const gpa_quad_problem* problem, const gpa_quad_grads* grads,
                                          hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_quad(problem)) return rc;
  if (!grads || !grads->dout || !grads->dx || !grads->u || !grads->dab || !grads->dgain)
    return fail(GPA_HIP_EINVAL, "quad features backward: dout, dx, u, dab and dgain required");
  const gpa_quad_problem& p = *problem;
  const dim3 grid((unsigned)((p.rows + QR - 1) / QR), (unsigned)p.heads);
  if (p.dtype == GPA_DTYPE_BF16) {
    const size_t lds = q_lds_bytes<bf16_t>(p.dim, true);
    if (int rc = q_lds_attr(quad_bwd<bf16_t>, lds)) return rc;
    hipLaunchKernelGGL((quad_bwd<bf16_t>), grid, dim3(QT), lds, stream, p, *grads);
  } else {
    const size_t lds = q_lds_bytes<float>(p.dim, true);
    if (int rc = q_lds_attr(quad_bwd<float>, lds)) return rc;
    hipLaunchKernelGGL((quad_bwd<float>), grid, dim3(QT), lds, stream, p, *grads);
  }
  return check_launch("gpa_quad_features_backward");
}
