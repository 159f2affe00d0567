// Slot counts and base logits of one level (reference attention.py:196-204
// with the counts of :318-319):
//   counts[t] = count0 + sum_{t' <= t} w[t']                (float32)
//   logits[t] = scale * raw[t] + gain * log1p(counts[t])
// for every (batch, head, slot) column, without materialising the counts.
// The token axis is cut into tiles of 64; the forward sums each tile, scans
// the tile sums per column (the counts before every tile, kept for the
// backward), then scans inside the tiles while writing the logits.  The
// backward reverses it: d counts = gain dl / (1 + counts) per token (counts
// recomputed from the saved tile prefixes), tile sums of d counts, their
// reverse scan, and the reverse scan inside the tiles gives d w.  One thread
// per column; consecutive threads take consecutive slots, so every access is
// coalesced.
#include <hip/hip_runtime.h>

#include "gpa_common.h"
#include "gpa_hip.h"

namespace gpa {
namespace {

constexpr int CT = 64;    // tokens per tile
constexpr int CNT = 256;  // threads per block (one column each; widths <= 256)

struct Cols {
  int B, T, H, M, N;
  __device__ __forceinline__ Cols(const gpa_count_problem& p)
      : B(p.batch), T(p.tokens), H(p.heads), M(p.slots), N((p.tokens + CT - 1) / CT) {}
  __device__ __forceinline__ int64_t at(const gpa_operand& o, int b, int t, int h) const {
    return (int64_t)b * o.sb + (int64_t)t * o.st + (int64_t)h * o.sh;
  }
  // [B,H,N,M] tile arrays
  __device__ __forceinline__ int64_t tile(int b, int h, int n, int m) const {
    return (((int64_t)b * H + h) * N + n) * M + m;
  }
  // [B,T,H,M] contiguous float32 rows
  __device__ __forceinline__ int64_t row(int b, int t, int h, int m) const {
    return (((int64_t)b * T + t) * H + h) * M + m;
  }
};

template <typename E>
__device__ __forceinline__ float ld(const gpa_operand& o, int64_t i) {
  return to_f32(reinterpret_cast<const E*>(o.ptr)[i]);
}

// Tile sums of w: prefix[b,h,n,m] = sum over tile n (scanned in place later).
template <typename E>
__global__ __launch_bounds__(CNT) void count_tile_sums(gpa_count_problem p) {
  const Cols c(p);
  const int n = blockIdx.x, b = blockIdx.y / c.H, h = blockIdx.y % c.H, m = threadIdx.x;
  if (m >= c.M) return;
  const int t0 = n * CT, t1 = t0 + CT < c.T ? t0 + CT : c.T;
  float s = 0.f;
#pragma unroll 16
  for (int t = t0; t < t1; ++t) s += ld<E>(p.write, c.at(p.write, b, t, h) + m);
  p.prefix[c.tile(b, h, n, m)] = s;
}

// Exclusive scan of the tile sums per column, from count0; the final counts.
__global__ __launch_bounds__(CNT) void count_tile_scan(gpa_count_problem p) {
  const Cols c(p);
  const int64_t col = (int64_t)blockIdx.x * CNT + threadIdx.x;
  if (col >= (int64_t)c.B * c.H * c.M) return;
  const int m = col % c.M, bh = col / c.M, b = bh / c.H, h = bh % c.H;
  float run = p.count0[(int64_t)b * p.count0_sb + (int64_t)h * c.M + m];
  for (int n = 0; n < c.N; ++n) {
    const int64_t i = c.tile(b, h, n, m);
    const float s = p.prefix[i];
    p.prefix[i] = run;
    run += s;
  }
  p.final_count[((int64_t)b * c.H + h) * c.M + m] = run;
}

template <typename E>
__global__ __launch_bounds__(CNT) void count_logits_fwd(gpa_count_problem p) {
  const Cols c(p);
  const int n = blockIdx.x, b = blockIdx.y / c.H, h = blockIdx.y % c.H, m = threadIdx.x;
  if (m >= c.M) return;
  const int t0 = n * CT, t1 = t0 + CT < c.T ? t0 + CT : c.T;
  const float scale = p.scale[h], gain = p.gain[h];
  float run = p.prefix[c.tile(b, h, n, m)];
#pragma unroll 8
  for (int t = t0; t < t1; ++t) {
    run += ld<E>(p.write, c.at(p.write, b, t, h) + m);
    p.logits[c.row(b, t, h, m)] = scale * ld<E>(p.raw, c.at(p.raw, b, t, h) + m) + gain * log1pf(run);
  }
}

// Backward 1: d raw, the per-tile sums of d counts (into `tsum`) and the
// per-tile partial sums of d gain and d scale.
template <typename E>
__global__ __launch_bounds__(CNT) void count_bwd_tiles(gpa_count_problem p, gpa_count_grads g) {
  __shared__ float red[CNT / 64][2];
  const Cols c(p);
  const int n = blockIdx.x, b = blockIdx.y / c.H, h = blockIdx.y % c.H, m = threadIdx.x;
  const int t0 = n * CT, t1 = t0 + CT < c.T ? t0 + CT : c.T;
  const float scale = p.scale[h], gain = p.gain[h];
  float dgain = 0.f, dscale = 0.f;
  if (m < c.M) {
    float run = p.prefix[c.tile(b, h, n, m)], sd = 0.f;
#pragma unroll 8
    for (int t = t0; t < t1; ++t) {
      run += ld<E>(p.write, c.at(p.write, b, t, h) + m);
      const float dl = g.dlogits[c.row(b, t, h, m)];
      const float raw = ld<E>(p.raw, c.at(p.raw, b, t, h) + m);
      reinterpret_cast<E*>(g.draw.ptr)[c.at(g.draw, b, t, h) + m] = from_f32<E>(scale * dl);
      dgain += dl * log1pf(run);
      dscale += dl * raw;
      sd += gain * dl / (1.f + run);
    }
    g.tsum[c.tile(b, h, n, m)] = sd;
  }
  for (int o = 32; o >= 1; o >>= 1) {
    dgain += __shfl_xor(dgain, o);
    dscale += __shfl_xor(dscale, o);
  }
  if ((threadIdx.x & 63) == 0) {
    red[threadIdx.x >> 6][0] = dgain;
    red[threadIdx.x >> 6][1] = dscale;
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    float x = 0.f;
    for (int w = 0; w < CNT / 64; ++w) x += red[w][threadIdx.x];
    g.partials[(((int64_t)b * c.H + h) * c.N + n) * 2 + threadIdx.x] = x;
  }
}

// Backward 2: reverse exclusive scan of the tile sums per column (plus the
// final counts' gradient): tsum[n] becomes the d counts of every token after
// tile n; d count0 = the whole sum.
__global__ __launch_bounds__(CNT) void count_bwd_scan(gpa_count_problem p, gpa_count_grads g) {
  const Cols c(p);
  const int64_t col = (int64_t)blockIdx.x * CNT + threadIdx.x;
  if (col >= (int64_t)c.B * c.H * c.M) return;
  const int m = col % c.M, bh = col / c.M, b = bh / c.H, h = bh % c.H;
  const int64_t f = ((int64_t)b * c.H + h) * c.M + m;
  float run = g.dfinal ? g.dfinal[f] : 0.f;
  for (int n = c.N - 1; n >= 0; --n) {
    const int64_t i = c.tile(b, h, n, m);
    const float s = g.tsum[i];
    g.tsum[i] = run;
    run += s;
  }
  if (g.dcount0) g.dcount0[f] = run;
}

// Backward 3: d w[t] = sum over t' >= t of d counts[t'] (reverse scan in the tile).
template <typename E>
__global__ __launch_bounds__(CNT) void count_bwd_write(gpa_count_problem p, gpa_count_grads g) {
  const Cols c(p);
  const int n = blockIdx.x, b = blockIdx.y / c.H, h = blockIdx.y % c.H, m = threadIdx.x;
  if (m >= c.M) return;
  const int t0 = n * CT, len = (t0 + CT < c.T ? t0 + CT : c.T) - t0;
  const float gain = p.gain[h];
  float dc[CT];
  float run = p.prefix[c.tile(b, h, n, m)];
  // Groups of 16 tokens: the loads of a group (at clamped tokens) are all
  // issued before the running sum uses them.
  constexpr int CG = 16;
#pragma unroll
  for (int i0 = 0; i0 < CT; i0 += CG) {
    float wv[CG], dl[CG];
#pragma unroll
    for (int j = 0; j < CG; ++j) {
      const int t = t0 + (i0 + j < len ? i0 + j : 0);
      wv[j] = ld<E>(p.write, c.at(p.write, b, t, h) + m);
      dl[j] = g.dlogits[c.row(b, t, h, m)];
    }
#pragma unroll
    for (int j = 0; j < CG; ++j) {
      const int i = i0 + j;
      dc[i] = 0.f;
      if (i < len) {
        run += wv[j];
        dc[i] = gain * dl[j] / (1.f + run);
      }
    }
  }
  float acc = g.tsum[c.tile(b, h, n, m)];
#pragma unroll
  for (int i = CT - 1; i >= 0; --i) {
    if (i < len) {
      acc += dc[i];
      reinterpret_cast<E*>(g.dwrite.ptr)[c.at(g.dwrite, b, t0 + i, h) + m] = from_f32<E>(acc);
    }
  }
}

int check_count(const gpa_count_problem* p) {
  if (!p) return fail(GPA_HIP_EINVAL, "count: null problem");
  if (p->batch < 1 || p->tokens < 1 || p->heads < 1 || p->slots < 1)
    return fail(GPA_HIP_EINVAL, "count: empty shape");
  if (p->slots > CNT) return fail(GPA_HIP_EUNSUPPORTED, "count: slot width above 256");
  if (p->dtype != GPA_DTYPE_F32 && p->dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "count: dtype");
  if (!p->raw.ptr || !p->write.ptr || !p->count0 || !p->gain || !p->scale || !p->prefix)
    return fail(GPA_HIP_EINVAL, "count: null pointer");
  return GPA_HIP_OK;
}

}  // namespace
}  // namespace gpa

extern "C" int gpa_count_logits_forward(const gpa_count_problem* problem, hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_count(problem)) return rc;
  if (!problem->logits || !problem->final_count) return fail(GPA_HIP_EINVAL, "count: null output");
  const gpa_count_problem& p = *problem;
  const dim3 tiles((p.tokens + CT - 1) / CT, p.batch * p.heads);
  const dim3 cols((unsigned)(((int64_t)p.batch * p.heads * p.slots + CNT - 1) / CNT));
  const bool bf = p.dtype == GPA_DTYPE_BF16;
  if (bf) hipLaunchKernelGGL(count_tile_sums<bf16_t>, tiles, dim3(CNT), 0, stream, p);
  else hipLaunchKernelGGL(count_tile_sums<float>, tiles, dim3(CNT), 0, stream, p);
  hipLaunchKernelGGL(count_tile_scan, cols, dim3(CNT), 0, stream, p);
  if (bf) hipLaunchKernelGGL(count_logits_fwd<bf16_t>, tiles, dim3(CNT), 0, stream, p);
  else hipLaunchKernelGGL(count_logits_fwd<float>, tiles, dim3(CNT), 0, stream, p);
  return check_launch("gpa_count_logits_forward");
}

extern "C" int gpa_count_logits_backward(const gpa_count_problem* problem, const gpa_count_grads* grads,
                                         hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_count(problem)) return rc;
  if (!grads || !grads->dlogits || !grads->draw.ptr || !grads->dwrite.ptr || !grads->partials || !grads->tsum)
    return fail(GPA_HIP_EINVAL, "count: null gradient buffer");
  const gpa_count_problem& p = *problem;
  const dim3 tiles((p.tokens + CT - 1) / CT, p.batch * p.heads);
  const dim3 cols((unsigned)(((int64_t)p.batch * p.heads * p.slots + CNT - 1) / CNT));
  const bool bf = p.dtype == GPA_DTYPE_BF16;
  if (bf) hipLaunchKernelGGL(count_bwd_tiles<bf16_t>, tiles, dim3(CNT), 0, stream, p, *grads);
  else hipLaunchKernelGGL(count_bwd_tiles<float>, tiles, dim3(CNT), 0, stream, p, *grads);
  hipLaunchKernelGGL(count_bwd_scan, cols, dim3(CNT), 0, stream, p, *grads);
  if (bf) hipLaunchKernelGGL(count_bwd_write<bf16_t>, tiles, dim3(CNT), 0, stream, p, *grads);
  else hipLaunchKernelGGL(count_bwd_write<float>, tiles, dim3(CNT), 0, stream, p, *grads);
  return check_launch("gpa_count_logits_backward");
}
