// One-token level write and residual (inference decode): reference
// src/gpa/attention.py:314-329 (_block_segment) and :190-194 (_residual) for a
// single token of every stream, from the block snapshots A^ [Dk][M] and
// B^ [M][Dv]:
//
//   w = softmax(u(key) A^), rounded to the activation type (the write)
//   key'   = key   - eta0 round(A^ w)
//   value' = value - eta1 round(w^T B^)
//
// One 256-thread workgroup per stream.  The logits and w^T B^ are column sums
// over rows (threads own a column; when the width is below 256 the rows are
// split between thread groups and the partial sums meet in LDS); A^ w is a
// row dot product per wave, eight rows at a time.  HBM bound: A^ is read
// twice (the second time mostly from cache), B^ once.
#include "token_step.h"

namespace gpa {
namespace {

constexpr int QNT = 256;  // threads per workgroup; every width is at most 256

template <typename E>
__global__ __launch_bounds__(QNT) void level_token(gpa_level_problem p) {
  __shared__ float uk[QNT], wf[QNT], zs[QNT], zp[QNT], rks[QNT];
  __shared__ float red[4], soft[2];
  const int s = blockIdx.x, b = s / p.heads, h = s - b * p.heads;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int Dk = p.key_dim, Dv = p.value_dim, M = p.slots;
  const float* A = p.a_first + (int64_t)b * p.a_first_sb + (int64_t)h * Dk * M;   // [Dk][M]
  const float* Bh = p.b_first + (int64_t)b * p.b_first_sb + (int64_t)h * M * Dv;  // [M][Dv]
  const E* key = reinterpret_cast<const E*>(p.key.ptr) + op_base(p.key, b, h);
  const E* val = reinterpret_cast<const E*>(p.value.ptr) + op_base(p.value, b, h);
  const float eta0 = p.eta[2 * h], eta1 = p.eta[2 * h + 1];

  // u(key) = key / max(||key||, 1e-6) in float32, rounded to the activation type.
  const float xk = t < Dk ? to_f32(key[t < Dk ? t : 0]) : 0.f;
  const float sk = sum64(xk * xk);
  if (lane == 0) red[wave] = sk;
  lds_barrier();
  const float nk = fmaxf(sqrtf(red[0] + red[1] + red[2] + red[3]), 1e-6f);
  if (t < Dk) uk[t] = round_as<E>(xk / nk);
  lds_barrier();

  // Logits z[m] = sum_k u(key)[k] A^[k][m]: thread (part, col), rows part + P i.
  {
    const int P = QNT / M, col = t % M, part = t / M;
    float z = 0.f;
    if (part < P) {
#pragma unroll 8
      for (int k = part; k < Dk; k += P) z += uk[k] * A[(int64_t)k * M + col];
    }
    zp[t] = z;
    lds_barrier();
    if (t < M) {
      float zt = 0.f;
      for (int q = 0; q < P; ++q) zt += zp[q * M + t];
      zs[t] = zt;
    }
    lds_barrier();
  }

  // Softmax over the M logits; the write is rounded to the activation type.
  if (wave == 0) {
    float mx = -INFINITY;
    for (int m = lane; m < M; m += 64) mx = fmaxf(mx, zs[m]);
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    float sm = 0.f;
    for (int m = lane; m < M; m += 64) sm += expf(zs[m] - mx);
    sm = sum64(sm);
    if (lane == 0) {
      soft[0] = mx;
      soft[1] = sm;
    }
  }
  lds_barrier();
  if (t < M) {
    const float w = round_as<E>(expf(zs[t] - soft[0]) / soft[1]);
    wf[t] = w;
    reinterpret_cast<E*>(p.write.ptr)[op_base(p.write, b, h) + t] = from_f32<E>(w);
  }
  lds_barrier();

  // rk[k] = sum_m A^[k][m] w[m]: wave `wave` takes rows wave + 4 r, eight rows
  // per pass with every load of the pass issued before the sums.
  for (int k0 = wave; k0 < Dk; k0 += 4 * 8) {
    float acc[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) acc[r] = 0.f;
    for (int m = lane; m < M; m += 64) {
      const float w = wf[m];
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int k = k0 + 4 * r;
        acc[r] += A[(int64_t)(k < Dk ? k : 0) * M + m] * w;
      }
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const float v = sum64(acc[r]);
      const int k = k0 + 4 * r;
      if (lane == 0 && k < Dk) rks[k] = v;
    }
  }

  // rv[v] = sum_m w[m] B^[m][v]: thread (part, col), rows part + P2 i.
  {
    const int P2 = QNT / Dv, col = t % Dv, part = t / Dv;
    float acc = 0.f;
    if (part < P2) {
#pragma unroll 8
      for (int m = part; m < M; m += P2) acc += wf[m] * Bh[(int64_t)m * Dv + col];
    }
    zp[t] = acc;
  }
  lds_barrier();
  if (t < Dv) {
    const int P2 = QNT / Dv;
    float rv = 0.f;
    for (int q = 0; q < P2; ++q) rv += zp[q * Dv + t];
    const float v = to_f32(val[t]);
    reinterpret_cast<E*>(p.value_out.ptr)[op_base(p.value_out, b, h) + t] = from_f32<E>(v - eta1 * round_as<E>(rv));
  }
  if (t < Dk) {
    reinterpret_cast<E*>(p.key_out.ptr)[op_base(p.key_out, b, h) + t] =
        from_f32<E>(xk - eta0 * round_as<E>(rks[t]));
  }
}


// The same step with every snapshot value in registers: all loads of the
// workgroup (A^ and B^ as float4 pieces) are issued before the first sum, so
// each stream costs one memory round trip.  Thread t holds the float4 column
// group t % (M/4) of A^ rows t / (M/4) + i NT/(M/4) and the group t % (Dv/4) of
// B^ rows t / (Dv/4) + i NT/(Dv/4) (i < RQ).  Widths multiples of 4 with
// (M/4) and (Dv/4) dividing NT, Dk M / 4 and M Dv / 4 at most RQ NT.
constexpr int RQ = 8;  // float4 pieces of A^ (and of B^) per thread

// RESID false: the write alone (key_out and value_out null: the last level,
// whose residual nothing reads): B^ is not loaded and neither product is formed.
template <typename E, int NT, bool RESID = true>
__device__ __forceinline__ void level_token_reg_run(const gpa_level_problem& p, int s) {
  constexpr int NW = NT / 64;
  __shared__ float uk[256], wf[256], zp[NT * 4], rks[256];
  __shared__ float red[NW], soft[2];
  const int b = s / p.heads, h = s - b * p.heads;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int Dk = p.key_dim, Dv = p.value_dim, M = p.slots;
  const int ga = M / 4, gb = Dv / 4;          // float4 groups per row
  const int ra = NT / ga, rb = NT / gb;       // rows per pass
  const int ca = t % ga, cb = t % gb;
  const float4* A = reinterpret_cast<const float4*>(p.a_first + (int64_t)b * p.a_first_sb + (int64_t)h * Dk * M);
  const float4* Bh = reinterpret_cast<const float4*>(p.b_first + (int64_t)b * p.b_first_sb + (int64_t)h * M * Dv);
  const E* key = reinterpret_cast<const E*>(p.key.ptr) + op_base(p.key, b, h);
  const E* val = reinterpret_cast<const E*>(p.value.ptr) + op_base(p.value, b, h);
  const int na = Dk * ga, nb = M * gb;       // float4 pieces of each snapshot
  float4 av[RQ], bv[RQ];
#pragma unroll
  for (int i = 0; i < RQ; ++i) {
    const int fa = t + NT * i, fb = t + NT * i;
    av[i] = A[fa < na ? fa : 0];
    if constexpr (RESID) bv[i] = Bh[fb < nb ? fb : 0];
  }
  const float xk = t < Dk ? to_f32(key[t < Dk ? t : 0]) : 0.f;
  const float xv = t < Dv ? to_f32(val[t < Dv ? t : 0]) : 0.f;
  const float eta0 = p.eta[2 * h], eta1 = p.eta[2 * h + 1];

  // u(key) = key / max(||key||, 1e-6) in float32, rounded to the activation type.
  const float sk = sum64(xk * xk);
  if (lane == 0) red[wave] = sk;
  __syncthreads();
  float nk2 = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) nk2 += red[w];
  const float nk = fmaxf(sqrtf(nk2), 1e-6f);
  if (t < Dk) uk[t] = round_as<E>(xk / nk);
  __syncthreads();

  // Logits z[m] = sum_k u(key)[k] A^[k][m]: partials over the thread's rows,
  // then over the ra threads of a column group.
  {
    float z0 = 0.f, z1 = 0.f, z2 = 0.f, z3 = 0.f;
#pragma unroll
    for (int i = 0; i < RQ; ++i) {
      const int row = t / ga + ra * i;
      if (row < Dk) {
        const float u = uk[row];
        z0 += u * av[i].x; z1 += u * av[i].y; z2 += u * av[i].z; z3 += u * av[i].w;
      }
    }
    const int part = t / ga;
    *reinterpret_cast<float4*>(&zp[part * M + 4 * ca]) = make_float4(z0, z1, z2, z3);
    __syncthreads();
    if (t < M) {
      float zt = 0.f;
      for (int q = 0; q < ra; ++q) zt += zp[q * M + t];
      wf[t] = zt;
    }
    __syncthreads();
  }

  // Softmax over the M logits; the write is rounded to the activation type.
  if (wave == 0) {
    float mx = -INFINITY;
    for (int m = lane; m < M; m += 64) mx = fmaxf(mx, wf[m]);
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    float sm = 0.f;
    for (int m = lane; m < M; m += 64) sm += expf(wf[m] - mx);
    sm = sum64(sm);
    if (lane == 0) {
      soft[0] = mx;
      soft[1] = sm;
    }
  }
  __syncthreads();
  float wt = 0.f;
  if (t < M) {
    wt = round_as<E>(expf(wf[t] - soft[0]) / soft[1]);
    reinterpret_cast<E*>(p.write.ptr)[op_base(p.write, b, h) + t] = from_f32<E>(wt);
  }
  if constexpr (!RESID) return;
  __syncthreads();  // every thread has read wf[t] for the softmax before it is overwritten
  if (t < M) wf[t] = wt;
  __syncthreads();

  // rk[k] = sum_m A^[k][m] w[m]: each row's ga column groups are ga
  // consecutive lanes (32 or 64) of one wave.
  {
    const float4 w4 = *reinterpret_cast<const float4*>(&wf[4 * ca]);
#pragma unroll
    for (int i = 0; i < RQ; ++i) {
      float d = av[i].x * w4.x + av[i].y * w4.y + av[i].z * w4.z + av[i].w * w4.w;
      for (int o = ga >> 1; o >= 1; o >>= 1) d += __shfl_xor(d, o, 64);
      const int row = t / ga + ra * i;
      if (ca == 0 && row < Dk) rks[row] = d;
    }
  }
  // rv[v] = sum_m w[m] B^[m][v]: partials over the thread's rows, then over
  // the rb threads of a column group.
  {
    float r0 = 0.f, r1 = 0.f, r2 = 0.f, r3 = 0.f;
#pragma unroll
    for (int i = 0; i < RQ; ++i) {
      const int row = t / gb + rb * i;
      if (row < M) {
        const float w = wf[row];
        r0 += w * bv[i].x; r1 += w * bv[i].y; r2 += w * bv[i].z; r3 += w * bv[i].w;
      }
    }
    __syncthreads();  // zp's logit partials are no longer read
    *reinterpret_cast<float4*>(&zp[(t / gb) * Dv + 4 * cb]) = make_float4(r0, r1, r2, r3);
  }
  __syncthreads();
  if (t < Dv) {
    float rv = 0.f;
    for (int q = 0; q < rb; ++q) rv += zp[q * Dv + t];
    reinterpret_cast<E*>(p.value_out.ptr)[op_base(p.value_out, b, h) + t] = from_f32<E>(xv - eta1 * round_as<E>(rv));
  }
  if (t < Dk)
    reinterpret_cast<E*>(p.key_out.ptr)[op_base(p.key_out, b, h) + t] = from_f32<E>(xk - eta0 * round_as<E>(rks[t]));
}

template <typename E, int NT, bool RESID>
__global__ __launch_bounds__(NT) void level_token_reg(gpa_level_problem p) {
  level_token_reg_run<E, NT, RESID>(p, blockIdx.x);
}

// A one-token step whose value and gates are formed in it (gpa_token_slot_step).
template <int NI>
__global__ __launch_bounds__(SNT) void gdn_token_slot_step(gpa_gdn_problem p, gpa_token_slot ts, float* fin,
                                                           gpa_operand out) {
  __shared__ TokenLds<NI> lds;
  token_run<bf16_t, NI, true>(p, fin, out, blockIdx.x, threadIdx.x, lds, ts);
}

// A level's inner one-token step (K <= 16 NI, every NT / 256 consecutive
// step workgroups in one NT-thread workgroup) and its one-token level write
// (one stream per workgroup) in one launch.  They share no buffers: the step
// reads the running state and writes a new one, the level write reads the
// block snapshots.  Step and level workgroups alternate while both last, so
// that each compute unit streams both kinds of data at once.
template <typename E, int NI, int NT, bool RESID = true, bool SLOT = false>
__global__ __launch_bounds__(NT) void token_level(gpa_gdn_problem sp, float* fin, gpa_operand out,
                                                  gpa_level_problem lp, int nstep, gpa_token_slot ts) {
  __shared__ TokenLds<NI> tl[NT / SNT];
  const int nlev = lp.batch * lp.heads, blk = blockIdx.x, both = nstep < nlev ? nstep : nlev;
  bool step;
  int idx;
  if (blk < 2 * both) {
    step = (blk & 1) == 0;
    idx = blk >> 1;
  } else {
    step = nstep > nlev;
    idx = blk - both;
  }
  if (!step) {
    level_token_reg_run<E, NT, RESID>(lp, idx);
    return;
  }
  const int u = threadIdx.x / SNT;
  token_run<E, NI, SLOT>(sp, fin, out, idx * (NT / SNT) + u, threadIdx.x % SNT, tl[u], ts);
}

// Threads for the register kernel (0: the shape is not covered).
int reg_threads(const gpa_level_problem& p) {
  const int Dk = p.key_dim, Dv = p.value_dim, M = p.slots;
  if (M % 4 || Dv % 4 || (reinterpret_cast<uintptr_t>(p.a_first) | reinterpret_cast<uintptr_t>(p.b_first)) % 16 ||
      p.a_first_sb % 4 || p.b_first_sb % 4)
    return 0;
  // (more threads with fewer pieces each: more waves in flight per compute unit)
  for (int nt : {256, 512, 1024}) {
    if (nt % (M / 4) || nt % (Dv / 4)) continue;
    if ((int64_t)Dk * M / 4 <= (int64_t)RQ * nt && (int64_t)M * Dv / 4 <= (int64_t)RQ * nt) return nt;
  }
  return 0;
}
int check_level_token(const gpa_level_problem* problem) {
  if (!problem) return fail(GPA_HIP_EINVAL, "level token: null problem");
  const gpa_level_problem& p = *problem;
  if (p.tokens != 1) return fail(GPA_HIP_EINVAL, "level token: needs tokens == 1");
  if (p.batch < 1 || p.heads < 1) return fail(GPA_HIP_EINVAL, "level token: empty shape");
  if (p.key_dim < 1 || p.key_dim > QNT || p.value_dim < 1 || p.value_dim > QNT || p.slots < 1 || p.slots > QNT)
    return fail(GPA_HIP_EUNSUPPORTED, "level token: key, value and slot widths must be in [1, 256]");
  if (p.dtype != GPA_DTYPE_F32 && p.dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "level token: dtype");
  if (!p.key.ptr || !p.value.ptr || !p.a_first || !p.b_first || !p.eta || !p.write.ptr)
    return fail(GPA_HIP_EINVAL, "level token: null pointer (the snapshots a_first and b_first are required)");
  if (!p.key_out.ptr != !p.value_out.ptr)
    return fail(GPA_HIP_EINVAL, "level token: key_out and value_out are both given or both null (write only)");
  if (p.given_write) return fail(GPA_HIP_EUNSUPPORTED, "level token: the one-token kernels form their own write");
  return GPA_HIP_OK;
}

}  // namespace
}  // namespace gpa

extern "C" int gpa_level_token_forward(const gpa_level_problem* problem, hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_level_token(problem)) return rc;
  const gpa_level_problem& p = *problem;
  const dim3 grid((unsigned)((int64_t)p.batch * p.heads));
  const bool bf = p.dtype == GPA_DTYPE_BF16, resid = p.key_out.ptr != nullptr;
  const int nt = reg_threads(p);
#define GPA_LEVEL_REG(NT)                                                                                   \
  do {                                                                                                      \
    if (bf && resid) hipLaunchKernelGGL((level_token_reg<bf16_t, NT, true>), grid, dim3(NT), 0, stream, p);  \
    else if (bf) hipLaunchKernelGGL((level_token_reg<bf16_t, NT, false>), grid, dim3(NT), 0, stream, p);   \
    else if (resid) hipLaunchKernelGGL((level_token_reg<float, NT, true>), grid, dim3(NT), 0, stream, p);  \
    else hipLaunchKernelGGL((level_token_reg<float, NT, false>), grid, dim3(NT), 0, stream, p);            \
  } while (0)
  if (nt == 256) GPA_LEVEL_REG(256);
  else if (nt == 512) GPA_LEVEL_REG(512);
  else if (nt == 1024) GPA_LEVEL_REG(1024);
  else if (!resid) return fail(GPA_HIP_EUNSUPPORTED, "level token: the write-only form needs the register kernel");
  else if (bf) hipLaunchKernelGGL(level_token<bf16_t>, grid, dim3(QNT), 0, stream, p);
  else hipLaunchKernelGGL(level_token<float>, grid, dim3(QNT), 0, stream, p);
#undef GPA_LEVEL_REG
  return check_launch("gpa_level_token_forward");
}

namespace gpa {
namespace {

// The one-launch form of a step and its level write (token_level), or -1
// where the shapes take two launches.  Only the 512-thread level kernel (M
// <= 128 at Dk = Dv = 128).  At 1024 threads (M = 256) the one launch is
// slower than the two: with the residual the step role's registers leave
// room for one workgroup per compute unit, and the write-only form measured
// 12-25 us slower too.
int launch_token_level(const gpa_gdn_problem& step, float* final_state, gpa_operand out,
                       const gpa_level_problem& level, const gpa_token_slot* ts, hipStream_t stream) {
  const int nt = reg_threads(level), ni = token_rows(step);
  const int64_t swg = token_workgroups(step), nlev = (int64_t)level.batch * level.heads;
  const bool resid = level.key_out.ptr != nullptr;
  const bool fused = step.dtype == level.dtype && nt == 512 && (ni == 8 || ni == 16) &&
                     swg % (nt / SNT) == 0 && swg / (nt / SNT) + nlev <= INT32_MAX / 2;
  if (!fused) return -1;
  const int nstep = (int)(swg / (nt / SNT));
  const dim3 grid((unsigned)(nstep + nlev));
  const bool bf = step.dtype == GPA_DTYPE_BF16;
  const gpa_token_slot none{};
#define GPA_TOKEN_LEVEL(E, NI, R, S)                                                                      \
  hipLaunchKernelGGL((token_level<E, NI, 512, R, S>), grid, dim3(512), 0, stream, step, final_state, out, \
                     level, nstep, ts ? *ts : none)
#define GPA_TOKEN_LEVEL_R(E, NI, S) \
  do { if (resid) GPA_TOKEN_LEVEL(E, NI, true, S); else GPA_TOKEN_LEVEL(E, NI, false, S); } while (0)
  if (ts) {  // bf16 only
    if (ni == 8) GPA_TOKEN_LEVEL_R(bf16_t, 8, true); else GPA_TOKEN_LEVEL_R(bf16_t, 16, true);
  } else if (bf) {
    if (ni == 8) GPA_TOKEN_LEVEL_R(bf16_t, 8, false); else GPA_TOKEN_LEVEL_R(bf16_t, 16, false);
  } else {
    if (ni == 8) GPA_TOKEN_LEVEL_R(float, 8, false); else GPA_TOKEN_LEVEL_R(float, 16, false);
  }
#undef GPA_TOKEN_LEVEL_R
#undef GPA_TOKEN_LEVEL
  return 0;
}

// A slot-in-step call's checks; `sp` is the step problem with stand-ins for
// v, g and beta (not read) so that check_token takes it.
int check_token_slot(const gpa_gdn_problem* step, const gpa_token_slot* ts, gpa_gdn_problem& sp) {
  if (!step || !ts) return fail(GPA_HIP_EINVAL, "slot step: null problem");
  sp = *step;
  if (sp.dtype != GPA_DTYPE_BF16) return fail(GPA_HIP_EUNSUPPORTED, "slot step: bf16 activations only");
  if (!sp.k.ptr) return fail(GPA_HIP_EINVAL, "slot step: needs a key (an update)");
  if (sp.kdim < 1 || sp.kdim > 256 || sp.kdim % (sp.kdim > 128 ? 64 : 32))
    return fail(GPA_HIP_EUNSUPPORTED, "slot step: K a multiple of 32 up to 128, or of 64 up to 256");
  if (!ts->center || !ts->gate_w || !ts->slot.ptr || !ts->gates.bias || !ts->gates.g_in || !ts->gates.b_in ||
      !ts->gates.g_out || !ts->gates.b_out)
    return fail(GPA_HIP_EINVAL, "slot step: null center, gate weight, bias or output");
  if (reinterpret_cast<uintptr_t>(ts->center) % 16)
    return fail(GPA_HIP_EINVAL, "slot step: center must be 16-byte aligned");
  sp.v = ts->slot;
  sp.g.ptr = ts->gates.g_in;
  sp.beta.ptr = ts->gates.b_in;
  return GPA_HIP_OK;
}

void launch_slot_step(const gpa_gdn_problem& sp, const gpa_token_slot& ts, float* final_state, gpa_operand out,
                      hipStream_t stream) {
  const dim3 grid((unsigned)token_workgroups(sp));
  switch (token_rows(sp)) {
    case 4: hipLaunchKernelGGL((gdn_token_slot_step<4>), grid, dim3(SNT), 0, stream, sp, ts, final_state, out); break;
    case 8: hipLaunchKernelGGL((gdn_token_slot_step<8>), grid, dim3(SNT), 0, stream, sp, ts, final_state, out); break;
    default: hipLaunchKernelGGL((gdn_token_slot_step<16>), grid, dim3(SNT), 0, stream, sp, ts, final_state, out);
  }
}

}  // namespace
}  // namespace gpa

extern "C" int gpa_token_level_forward(const gpa_gdn_problem* step, float* final_state, gpa_operand out,
                                       const gpa_level_problem* level, hipStream_t stream) {
  using namespace gpa;
  if (int rc = check_token(step, final_state, out)) return rc;
  if (int rc = check_level_token(level)) return rc;
  if (launch_token_level(*step, final_state, out, *level, nullptr, stream) < 0) {
    if (int rc = gpa_gdn_token_step(step, final_state, out, stream)) return rc;
    return gpa_level_token_forward(level, stream);
  }
  return check_launch("gpa_token_level_forward");
}

extern "C" int gpa_token_slot_step(const gpa_gdn_problem* step, const gpa_token_slot* slot, float* final_state,
                                   gpa_operand out, const gpa_level_problem* level, hipStream_t stream) {
  using namespace gpa;
  gpa_gdn_problem sp;
  if (int rc = check_token_slot(step, slot, sp)) return rc;
  if (int rc = check_token(&sp, final_state, out)) return rc;
  if (level) {
    if (int rc = check_level_token(level)) return rc;
    if (launch_token_level(sp, final_state, out, *level, slot, stream) == 0)
      return check_launch("gpa_token_slot_step");
  }
  launch_slot_step(sp, *slot, final_state, out, stream);
  if (int rc = check_launch("gpa_token_slot_step")) return rc;
  return level ? gpa_level_token_forward(level, stream) : GPA_HIP_OK;
}
