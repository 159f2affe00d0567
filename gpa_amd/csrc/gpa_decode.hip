// Batched single-token decode step of the DenseGPA core: one workgroup of 256
// threads per (b, h) stream does, for its token, everything the reference's
// chunk-mode block segment does at T = 1 (src/gpa/attention.py:299-345):
//   per level j:  slot = key C_j^T, gates from u(key) W_j + b_j,
//                 inner GDN step on A_j with read raw_j = u(q)^T A_j,
//                 write a_j = softmax(u(key) A^_j), counts, logits,
//                 residual key -= eta A^_j a_j, value -= eta a_j^T B^_j
//   per edge e = (i -> j): GDN step on R_e, message u(p_i)^T R_e
//   per level j:  route reader (attention.py:225-262), then the outer GDN step
//                 on B_j and its read with the route query
//   out = sum_j softmax_L(output_logits)_j o_j
// rounding to the activation type wherever the reference rounds.
//
// Memory.  Each state matrix (fp32 [rows][cols], per head contiguous) is read
// once and written once: 32-column blocks, 8 threads per column each holding
// an eighth of the rows in registers; the rank-1 update and the read happen
// in registers.  A^_j a_j is a transposed sum across the lanes of a half-wave.
// Parameters (shared by every batch element) are read through L2.
#include <hip/hip_runtime.h>

#include "gdn_common.h"

namespace gpa {
namespace {

constexpr int DT = 256;                  // threads per workgroup (4 waves: 512 VGPRs each)
constexpr int DWID = GPA_DECODE_MAX_WIDTH;
constexpr int PARTS = 8, COLS = DT / PARTS;
constexpr int RPT = DWID / PARTS;        // rows per thread of a state column block
constexpr int NL = GPA_DECODE_MAX_LEVELS, NE = GPA_DECODE_MAX_EDGES;

struct Smem {
  float qhat[DWID], key[DWID], val[DWID], kuh[DWID], out[DWID];
  float slot[NL][DWID], vlev[NL][DWID], wr[NL][DWID], loc[NL][DWID], lg[NL][DWID];
  float whn[NL][DWID], lhn[NL][DWID];  // u(write_i), u(local_i), rounded
  float gates[NL][4];
  float msg[NE][DWID];
  float red[PARTS][COLS];
  float va[2 * DWID], vb[2 * DWID], vc[DWID], vd[DWID];
  float rk[DWID], rv[DWID];
  float scal[8];
};

__device__ __forceinline__ float softplus(float x) { return x > 20.f ? x : log1pf(__expf(x)); }
__device__ __forceinline__ float sigmoidf(float x) { return 1.f / (1.f + __expf(-x)); }

// ---- wave 0 vector helpers (n <= 256); callers synchronise afterwards.
template <typename E>
__device__ void w0_unit(const float* x, float* y, int n) {
  const int lane = threadIdx.x & 63;
  float v[DWID / 64], ss = 0.f;
#pragma unroll
  for (int i = 0; i < DWID / 64; ++i) {
    const int d = lane + 64 * i;
    v[i] = d < n ? x[d] : 0.f;
    ss += v[i] * v[i];
  }
  const float den = fmaxf(sqrtf(sum64(ss)), 1e-6f);
#pragma unroll
  for (int i = 0; i < DWID / 64; ++i) {
    const int d = lane + 64 * i;
    if (d < n) y[d] = round_as<E>(v[i] / den);
  }
}

// softmax of n <= 256 values; y may alias x.  ROUND: round the result to E.
template <typename E, bool ROUND>
__device__ void w0_softmax(const float* x, float* y, int n) {
  const int lane = threadIdx.x & 63;
  float v[DWID / 64], m = -INFINITY;
#pragma unroll
  for (int i = 0; i < DWID / 64; ++i) {
    const int d = lane + 64 * i;
    v[i] = d < n ? x[d] : -INFINITY;
    m = fmaxf(m, v[i]);
  }
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < DWID / 64; ++i) {
    const int d = lane + 64 * i;
    v[i] = d < n ? __expf(v[i] - m) : 0.f;
    s += v[i];
  }
  s = sum64(s);
#pragma unroll
  for (int i = 0; i < DWID / 64; ++i) {
    const int d = lane + 64 * i;
    if (d < n) y[d] = ROUND ? round_as<E>(v[i] / s) : v[i] / s;
  }
}

__device__ __forceinline__ float part_sum(const float* red, int cl) {
  float s = 0.f;
#pragma unroll
  for (int q = 0; q < PARTS; ++q) s += red[q * COLS + cl];
  return s;
}

// Sums of a lane's 32 values over the 32 lanes of its half-wave by recursive
// halving; lane l returns the total of value index l % 32.
__device__ __forceinline__ float halfwave_transpose_sum(float (&v)[32], int lane) {
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) {
    const bool up = lane & m;
#pragma unroll
    for (int j = 0; j < m; ++j) {
      const float send = up ? v[j] : v[j + m], keep = up ? v[j + m] : v[j];
      v[j] = keep + __shfl_xor(send, m);
    }
  }
  return v[0];
}

// out[r] = round_E(sum_c vec[c] round_E(P[r][c])) for a parameter matrix with
// contiguous rows: wave w takes rows w, w + 4, ...; each lane holds up to 4
// columns; loads of 4 rows are issued before their reductions.
template <typename E>
__device__ void param_row_dots(const float* P, int rows, int cols, const float* vec, float* out) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int r0 = wave; r0 < rows; r0 += 16) {
    float x[4][DWID / 64];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = r0 + 4 * j, rr = r < rows ? r : rows - 1;
#pragma unroll
      for (int i = 0; i < DWID / 64; ++i) {
        const int c = lane + 64 * i;
        x[j][i] = P[rr * cols + (c < cols ? c : 0)];
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < DWID / 64; ++i) {
        const int c = lane + 64 * i;
        if (c < cols) acc += vec[c] * round_as<E>(x[j][i]);
      }
      acc = sum64(acc);
      const int r = r0 + 4 * j;
      if (lane == 0 && r < rows) out[r] = round_as<E>(acc);
    }
  }
}

// out[c] = sum_r vec[r] round_E(P[r][c]) (no rounding of the sum) for a
// row-major parameter matrix [R][C]; R, C <= 512.
template <typename E>
__device__ void param_col_reads(const float* P, int R, int C, const float* vec, float* out, float* red) {
  const int tid = threadIdx.x, part = tid / COLS, cl = tid % COLS;
  for (int c0 = 0; c0 < C; c0 += COLS) {
    const int c = c0 + cl, cc = c < C ? c : C - 1;
    float acc = 0.f;
#pragma unroll 8
    for (int r = part; r < R; r += PARTS) acc += vec[r] * round_as<E>(P[r * C + cc]);
    red[part * COLS + cl] = acc;
    __syncthreads();
    if (part == 0 && c < C) out[c] = part_sum(red, cl);
    __syncthreads();
  }
}

// out[c] = sum_r vec[r] S[r][c] for a state matrix [R][C] (R, C <= 256).
__device__ void state_col_reads(const float* S, int R, int C, const float* vec, float* out, float* red) {
  const int tid = threadIdx.x, part = tid / COLS, cl = tid % COLS;
  for (int c0 = 0; c0 < C; c0 += COLS) {
    const int c = c0 + cl, cc = c < C ? c : C - 1;
    float x[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int r = part + PARTS * i;
      x[i] = S[(r < R ? r : R - 1) * C + cc];  // 32-bit offsets: one VGPR per address
    }
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int r = part + PARTS * i;
      if (r < R) acc += vec[r] * x[i];
    }
    red[part * COLS + cl] = acc;
    __syncthreads();
    if (part == 0 && c < C) out[c] = part_sum(red, cl);
    __syncthreads();
  }
}

// One GDN step of a state S [R][C] (R, C <= 256):
//   S' = e^g S + beta khat (v - e^g khat^T S)^T,   y = qhat^T S'   (when y != NULL)
__device__ void state_step(const float* S, float* So, int R, int C, const float* khat, const float* vvec,
                           float g, float beta, const float* qhat, float* y, float* red) {
  const int tid = threadIdx.x, part = tid / COLS, cl = tid % COLS;
  const float eg = __expf(g);
  for (int c0 = 0; c0 < C; c0 += COLS) {
    const int c = c0 + cl;
    const bool cin = c < C;
    const int cc = cin ? c : C - 1;
    float x[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int r = part + PARTS * i;
      x[i] = S[(r < R ? r : R - 1) * C + cc];  // 32-bit offsets: one VGPR per address
    }
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int r = part + PARTS * i;
      if (r < R) d += khat[r] * x[i];
    }
    red[part * COLS + cl] = d;
    __syncthreads();
    const float err = vvec[cc] - eg * (part_sum(red, cl));
    float yy = 0.f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int r = part + PARTS * i;
      if (r < R) {
        const float xn = eg * x[i] + beta * khat[r] * err;
        if (cin) So[r * C + c] = xn;
        if (y) yy += qhat[r] * xn;
      }
    }
    __syncthreads();
    if (y) {
      red[part * COLS + cl] = yy;
      __syncthreads();
      if (part == 0 && cin) y[c] = part_sum(red, cl);
      __syncthreads();
    }
  }
}

// Block-start snapshot pass of a level (A^ [R = Dk][C = M]):
//   w = round_E(softmax(ku^T A^)),  rk = A^ w   (rk zeroed by the caller)
// Two reads of A^ (the second mostly from L2): the softmax needs every column
// before A^ w can start.
template <typename E>
__device__ void snapshot_write(const float* A, int R, int C, const float* ku, float* w, float* rk, float* red) {
  const int tid = threadIdx.x, part = tid / COLS, cl = tid % COLS, lane = tid & 63;
  state_col_reads(A, R, C, ku, w, red);
  if (tid < 64) w0_softmax<E, true>(w, w, C);
  __syncthreads();
  // A^ w, one column block at a time: lane l ends with row part + PARTS (l % 32)
  // summed over its half-wave's COLS columns.
  static_assert(COLS == 32 && RPT == 32, "one part per half-wave");
  const int r = part + PARTS * (lane & 31);
  for (int c0 = 0; c0 < C; c0 += COLS) {
    const int c = c0 + cl, cc = c < C ? c : C - 1;
    float x[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int rr = part + PARTS * i;
      x[i] = A[(rr < R ? rr : R - 1) * C + cc];
    }
    const float wc = c < C ? w[c] : 0.f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) x[i] *= wc;
    const float tot = halfwave_transpose_sum(x, lane);
    if (r < R) atomicAdd(&rk[r], tot);
  }
  __syncthreads();
}

// Per-level and per-edge descriptors copied from the kernel arguments with
// constant indices, so that the level and edge loops index LDS, not the
// argument block (a dynamic index into it would copy it to scratch).
struct Table {
  gpa_decode_level level[NL];
  gpa_decode_state relation[NE];
  float* relation_out[NE];
};

template <typename E>
__global__ __launch_bounds__(DT, 1) void gpa_decode_kernel(gpa_decode_problem p) {
  __shared__ Smem sm;
  __shared__ Table tab;
  if (threadIdx.x == 0) {
#pragma unroll
    for (int j = 0; j < NL; ++j) tab.level[j] = p.level[j];
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      tab.relation[e] = p.relation[e];
      tab.relation_out[e] = p.relation_out[e];
    }
  }
  const int s = blockIdx.x, b = s / p.heads, h = s % p.heads, H = p.heads;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int Dk = p.key_dim, Dv = p.value_dim, L = p.levels;
  auto act = [&](const gpa_operand& o, int d) {
    return to_f32(reinterpret_cast<const E*>(o.ptr)[(int64_t)b * o.sb + (int64_t)h * o.sh + d]);
  };
  auto state_at = [&](const gpa_decode_state& st, int rows, int cols) {
    return st.ptr + (int64_t)b * st.sb + (int64_t)h * rows * cols;
  };
  auto out_at = [&](float* o, int rows, int cols) { return o + ((int64_t)b * H + h) * rows * cols; };

  if (tid < Dk) sm.key[tid] = act(p.k, tid);
  if (tid < Dv) sm.val[tid] = act(p.v, tid);
  if (tid < Dk) sm.va[tid] = act(p.q, tid);
  if (tid < DWID) sm.out[tid] = 0.f;
  __syncthreads();
  if (wave == 0) w0_unit<E>(sm.va, sm.qhat, Dk);
  __syncthreads();

  // ---------------------------------------------------------------- levels
  for (int j = 0; j < L; ++j) {
    const gpa_decode_level& lv = tab.level[j];
    const int M = lv.slots;
    param_row_dots<E>(lv.center + (int64_t)h * M * Dk, M, Dk, sm.key, sm.slot[j]);
    if (wave == 0) w0_unit<E>(sm.key, sm.kuh, Dk);
    if (tid < DWID) sm.rk[tid] = 0.f;
    __syncthreads();
    if (wave == 0) {
      // gates: u(key) W (rounded) + bias
      const float* gw = lv.gate_weight + (int64_t)h * Dk * 4;
      float a[4] = {0.f, 0.f, 0.f, 0.f};
      for (int d = lane; d < Dk; d += 64)
#pragma unroll
        for (int c = 0; c < 4; ++c) a[c] += sm.kuh[d] * round_as<E>(gw[d * 4 + c]);
#pragma unroll
      for (int c = 0; c < 4; ++c) a[c] = round_as<E>(sum64(a[c])) + lv.gate_bias[h * 4 + c];
      if (lane == 0) {
        const bool none = p.positional_none != 0;
        sm.gates[j][0] = none ? 0.f : -fminf(softplus(a[0]), 10.f);
        sm.gates[j][1] = p.beta_max * sigmoidf(a[1]);
        sm.gates[j][2] = none ? 0.f : -fminf(softplus(a[2]), 10.f);
        sm.gates[j][3] = p.beta_max * sigmoidf(a[3]);
      }
    }
    __syncthreads();
    // inner step with its read raw_j = u(q)^T A_j
    state_step(state_at(lv.inner, Dk, M), out_at(lv.inner_out, Dk, M), Dk, M, sm.kuh, sm.slot[j],
               sm.gates[j][0], sm.gates[j][1], sm.qhat, sm.va, &sm.red[0][0]);
    // write a_j and A^_j a_j from the block-start snapshot
    snapshot_write<E>(state_at(lv.snap_inner, Dk, M), Dk, M, sm.kuh, sm.wr[j], sm.rk, &sm.red[0][0]);
    // counts and logits
    if (tid < M) {
      const float* cnt = lv.count.ptr + (int64_t)b * lv.count.sb + (int64_t)h * M;
      const float n = cnt[tid] + sm.wr[j][tid];
      lv.count_out[((int64_t)b * H + h) * M + tid] = n;
      const float gain = softplus(p.count_gain_raw[j * H + h]);
      sm.lg[j][tid] = p.read_scale * round_as<E>(sm.va[tid]) + gain * log1pf(n);
    }
    // a_j^T B^_j
    state_col_reads(state_at(lv.snap_outer, M, Dv), M, Dv, sm.wr[j], sm.rv, &sm.red[0][0]);
    // residuals (the outer step later uses this level's value before them)
    {
      const float e0 = 1.f + .25f * tanhf(p.residual_raw[(j * H + h) * 2]);
      const float e1 = 1.f + .25f * tanhf(p.residual_raw[(j * H + h) * 2 + 1]);
      if (tid < Dv) {
        sm.vlev[j][tid] = sm.val[tid];
        sm.val[tid] = round_as<E>(sm.val[tid] - e1 * round_as<E>(sm.rv[tid]));
      }
      if (tid < Dk) sm.key[tid] = round_as<E>(sm.key[tid] - e0 * round_as<E>(sm.rk[tid]));
    }
    __syncthreads();
  }

  // ---------------------------------------------------------------- relations
  for (int j = 0; j < L; ++j) {
    if (wave == 0) w0_softmax<E, true>(sm.lg[j], sm.loc[j], tab.level[j].slots);
  }
  __syncthreads();
  for (int j = 0; j < L; ++j) {
    if (wave == 0) w0_unit<E>(sm.wr[j], sm.whn[j], tab.level[j].slots);
    if (wave == 1) w0_unit<E>(sm.loc[j], sm.lhn[j], tab.level[j].slots);
  }
  __syncthreads();
  {
    int e = 0;
    for (int i = 0; i < L; ++i)
      for (int j = 0; j < L; ++j) {
        if (i == j) continue;
        const int Mi = tab.level[i].slots, Mj = tab.level[j].slots;
        const float g = p.positional_none ? 0.f : -softplus(p.relation_decay_raw[e * H + h]);
        const float beta = sigmoidf(p.relation_beta_raw[e * H + h]);
        state_step(state_at(tab.relation[e], Mi, Mj), out_at(tab.relation_out[e], Mi, Mj), Mi, Mj, sm.whn[i],
                   sm.wr[j], g, beta, sm.lhn[i], sm.msg[e], &sm.red[0][0]);
        if (tid < Mj) sm.msg[e][tid] = round_as<E>(sm.msg[e][tid]);
        __syncthreads();
        ++e;
      }
  }

  // ---------------------------------------------------------------- route reader and outer reads
  float lw = 0.f;  // 1 / sum_j e^{output_logits[j,h] - max}
  {
    float mx = -INFINITY;
    for (int j = 0; j < L; ++j) mx = fmaxf(mx, p.output_logits[j * H + h]);
    float den = 0.f;
    for (int j = 0; j < L; ++j) den += __expf(p.output_logits[j * H + h] - mx);
    lw = 1.f / den;
  }
  for (int j = 0; j < L; ++j) {
    const gpa_decode_level& lv = tab.level[j];
    const int M = lv.slots;
    // incoming messages: softmax over the edges into j
    if (tid < M) {
      float mx = -INFINITY;
      int e = 0;
      for (int i = 0; i < L; ++i)
        for (int t = 0; t < L; ++t) {
          if (i == t) continue;
          if (t == j) mx = fmaxf(mx, p.edge_logits[e * H + h]);
          ++e;
        }
      float den = 0.f, acc = 0.f;
      e = 0;
      for (int i = 0; i < L; ++i)
        for (int t = 0; t < L; ++t) {
          if (i == t) continue;
          if (t == j) {
            const float w = __expf(p.edge_logits[e * H + h] - mx);
            den += w;
            acc += w * sm.msg[e][tid];
          }
          ++e;
        }
      sm.vc[tid] = L > 1 ? acc / den : 0.f;
    }
    __syncthreads();
    if (wave == 0 && L > 1) {
      // centred, RMS-normalised, tanh-squashed incoming (legacy read)
      float v[DWID / 64], s1 = 0.f;
#pragma unroll
      for (int i = 0; i < DWID / 64; ++i) {
        const int d = lane + 64 * i;
        v[i] = d < M ? sm.vc[d] : 0.f;
        s1 += v[i];
      }
      const float mean = sum64(s1) / M;
      float s2 = 0.f;
#pragma unroll
      for (int i = 0; i < DWID / 64; ++i) {
        const int d = lane + 64 * i;
        v[i] = d < M ? v[i] - mean : 0.f;
        s2 += v[i] * v[i];
      }
      const float rms = sqrtf(sum64(s2) / M + 1e-5f);
      const float gain = p.relation_gain[j * H + h];
#pragma unroll
      for (int i = 0; i < DWID / 64; ++i) {
        const int d = lane + 64 * i;
        if (d < M) sm.vd[d] = sm.lg[j][d] + gain * tanhf(v[i] / rms);
      }
    } else if (wave == 0) {
      for (int d = lane; d < M; d += 64) sm.vd[d] = sm.lg[j][d];
    }
    __syncthreads();
    if (wave == 0) w0_softmax<E, true>(sm.vd, sm.vd, M);  // route
    __syncthreads();
    // route MLP: hidden = gelu(route U) (rounded), route += gain * hidden D
    param_col_reads<E>(lv.route_up + (int64_t)h * M * 2 * M, M, 2 * M, sm.vd, sm.va, &sm.red[0][0]);
    for (int i = tid; i < 2 * M; i += DT) {
      const float x = round_as<E>(sm.va[i]);
      sm.va[i] = round_as<E>(.5f * x * (1.f + erff(x * 0.70710678118654752f)));
    }
    __syncthreads();
    param_col_reads<E>(lv.route_down + (int64_t)h * 2 * M * M, 2 * M, M, sm.va, sm.vb, &sm.red[0][0]);
    if (tid < M) sm.vd[tid] = round_as<E>(sm.vd[tid] + p.route_mlp_gain[j * H + h] * round_as<E>(sm.vb[tid]));
    __syncthreads();
    // qo = route W_rs + query_scale q W_qs
    param_col_reads<E>(lv.route_weight + (int64_t)h * M * M, M, M, sm.vd, sm.va, &sm.red[0][0]);
    if (tid < Dk) sm.vc[tid] = act(p.q, tid);
    __syncthreads();
    param_col_reads<E>(lv.query_weight + (int64_t)h * Dk * M, Dk, M, sm.vc, sm.vb, &sm.red[0][0]);
    if (tid < M)
      sm.vc[tid] = round_as<E>(round_as<E>(sm.va[tid]) + round_as<E>(p.query_scale * round_as<E>(sm.vb[tid])));
    __syncthreads();
    if (wave == 0) w0_unit<E>(sm.vc, sm.vd, M);                 // u(qo)
    if (wave == 1) w0_unit<E>(sm.slot[j], sm.va, M);            // u(slot)
    __syncthreads();
    // outer step and its read with the route query
    state_step(state_at(lv.outer, M, Dv), out_at(lv.outer_out, M, Dv), M, Dv, sm.va, sm.vlev[j],
               sm.gates[j][2], sm.gates[j][3], sm.vd, sm.vb, &sm.red[0][0]);
    if (tid < Dv) {
      float mx = -INFINITY;
      for (int t = 0; t < L; ++t) mx = fmaxf(mx, p.output_logits[t * H + h]);
      const float w = __expf(p.output_logits[j * H + h] - mx) * lw;
      sm.out[tid] += w * round_as<E>(sm.vb[tid]);
    }
    __syncthreads();
  }
  if (tid < Dv) {
    E* o = reinterpret_cast<E*>(p.out.ptr);
    o[(int64_t)b * p.out.sb + (int64_t)h * p.out.sh + tid] = from_f32<E>(sm.out[tid]);
  }
}

int check_decode(const gpa_decode_problem* p) {
  if (!p) return fail(GPA_HIP_EINVAL, "decode: null problem");
  if (p->batch < 1 || p->heads < 1 || p->levels < 1 || p->levels > NL)
    return fail(GPA_HIP_EINVAL, "decode: batch, heads >= 1 and 1 <= levels <= 4");
  if (p->key_dim < 1 || p->key_dim > DWID || p->value_dim < 1 || p->value_dim > DWID)
    return fail(GPA_HIP_EUNSUPPORTED, "decode: key and value widths must be in [1, 256]");
  if (p->dtype != GPA_DTYPE_F32 && p->dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "decode: dtype");
  if (!p->q.ptr || !p->k.ptr || !p->v.ptr || !p->out.ptr) return fail(GPA_HIP_EINVAL, "decode: null q/k/v/out");
  for (int j = 0; j < p->levels; ++j) {
    const gpa_decode_level& lv = p->level[j];
    if (lv.slots < 1 || lv.slots > DWID) return fail(GPA_HIP_EUNSUPPORTED, "decode: slots must be in [1, 256]");
    if (!lv.center || !lv.gate_weight || !lv.gate_bias || !lv.route_weight || !lv.query_weight || !lv.route_up ||
        !lv.route_down || !lv.inner.ptr || !lv.outer.ptr || !lv.count.ptr || !lv.snap_inner.ptr ||
        !lv.snap_outer.ptr || !lv.inner_out || !lv.outer_out || !lv.count_out)
      return fail(GPA_HIP_EINVAL, "decode: a level pointer is null");
  }
  const int ne = p->levels * (p->levels - 1);
  for (int e = 0; e < ne; ++e)
    if (!p->relation[e].ptr || !p->relation_out[e]) return fail(GPA_HIP_EINVAL, "decode: a relation pointer is null");
  if (!p->residual_raw || !p->count_gain_raw || !p->route_mlp_gain || !p->output_logits || !p->relation_gain ||
      (ne && (!p->edge_logits || !p->relation_decay_raw || !p->relation_beta_raw)))
    return fail(GPA_HIP_EINVAL, "decode: a parameter pointer is null");
  if ((int64_t)p->batch * p->heads > 0x7fffffff) return fail(GPA_HIP_EUNSUPPORTED, "decode: too many streams");
  return GPA_HIP_OK;
}

}  // namespace
}  // namespace gpa

extern "C" int gpa_decode_step(const gpa_decode_problem* problem, hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_decode(problem)) return rc;
  const dim3 grid(problem->batch * problem->heads), block(DT);
  if (problem->dtype == GPA_DTYPE_BF16)
    hipLaunchKernelGGL(gpa_decode_kernel<bf16_t>, grid, block, 0, stream, *problem);
  else
    hipLaunchKernelGGL(gpa_decode_kernel<float>, grid, block, 0, stream, *problem);
  return check_launch("gpa_decode_step");
}
