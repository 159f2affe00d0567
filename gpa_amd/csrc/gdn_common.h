// Device helpers shared by the GDN scan kernels (gdn_scan.hip, gdn_state_mfma.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gpa_common.h"
#include "gpa_hip.h"

namespace gpa {

// bf16 pairs for the split (hi + lo) MFMA operands.  bf2_pack rounds two
// floats to bf16 (round to nearest even, one v_cvt_pk_bf16_f32), x0 in the
// low half; bf2_low / bf2_high widen a half back to float (exact).
// bf2_split gives hi = bf16(x) and lo = bf16(x - hi) of a pair, forming
// x - hi from the packed hi word: one shift or mask per value, where
// converting each hi element back costs a second rounding and a shift.
typedef __bf16 bf16pair_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf2_pack(float x0, float x1) {
  const bf16pair_t h = {(__bf16)x0, (__bf16)x1};
  uint32_t w;
  __builtin_memcpy(&w, &h, 4);
  return w;
}
// (The low half moves up through v_perm_b32, bytes 1:0 -> 3:2 over zeros, so
// that the compiler does not turn the shift back into a second rounding.)
__device__ __forceinline__ float bf2_low(uint32_t w) { return __uint_as_float(__builtin_amdgcn_perm(0u, w, 0x01000c0cu)); }
__device__ __forceinline__ float bf2_high(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ void bf2_split(float x0, float x1, uint32_t& hi, uint32_t& lo) {
  hi = bf2_pack(x0, x1);
  lo = bf2_pack(x0 - bf2_low(hi), x1 - bf2_high(hi));
}

constexpr int R = GPA_CHUNK_ROWS;  // rows per chunk tile
constexpr int NT = 256;            // threads per block
constexpr int VT = 32;             // state columns per sequential block
constexpr int KS = 64;             // staged K slice
constexpr int LDR = R + 1;         // padded row stride of R x R tiles
constexpr int LDS_ = KS + 1;       // padded row stride of R x KS tiles

// Barrier that orders LDS only.  __syncthreads() also waits for every
// outstanding global load and store of the wave (a workgroup-scope fence); a
// kernel whose waves exchange data through LDS alone, and which never reads
// back global memory it writes, keeps its global traffic in flight across
// this barrier.  The "memory" clobber keeps the compiler from moving LDS
// accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ int token_at(const gpa_gdn_problem& p, int n, int r) {
  if (r >= p.chunk) return -1;
  const int t = n * p.chunk + r - p.offset;
  return (t >= 0 && t < p.tokens) ? t : -1;
}

__device__ __forceinline__ int64_t op_base(const gpa_operand& o, int b, int h) {
  return (int64_t)b * o.sb + (int64_t)h * o.sh;
}

template <typename E>
__device__ __forceinline__ float op_load(const gpa_operand& o, int b, int h, int t, int d) {
  return to_f32(reinterpret_cast<const E*>(o.ptr)[op_base(o, b, h) + (int64_t)t * o.st + d]);
}

__device__ __forceinline__ float scalar_load(const gpa_operand& o, int b, int h, int t) {
  return reinterpret_cast<const float*>(o.ptr)[op_base(o, b, h) + (int64_t)t * o.st];
}

// Stream-major saved buffer offsets.
// [S][N][R][width] (position rows): kn, qn, w, dw, tri (width R), gam, beta (width 1)
__device__ __forceinline__ int64_t rows_off(int s, int n, int nch, int r, int width) {
  return (((int64_t)s * nch + n) * R + r) * width;
}
// [S][N][V][K] value-major chunk-start states: element (k,v) at +v*K+k
__device__ __forceinline__ int64_t state_off(int s, int n, int nch, int K, int V) {
  return ((int64_t)s * nch + n) * K * V;
}
// [S][N][V][R] value-major position data (u, delta, dd0, o, ddelta): (r,v) at +v*R+r
__device__ __forceinline__ int64_t vc_off(int s, int n, int nch, int V) {
  return ((int64_t)s * nch + n) * V * R;
}
// MFMA path: U in fragment order, per chunk [ceil(V/32)][2][4][64][4]: for
// 32-column strip c, row tile rt and group g, lane l holds U rows
// 32 rt + 8 g + 4 (l/32) + 0..3 of column 32 c + l%32 (the accumulator layout
// of a 32 x 32 MFMA tile), so a wave reads 1 KB contiguous per instruction.
__host__ __device__ __forceinline__ int ufrag_v(int V) { return (V + 31) / 32 * 32; }  // padded width
__device__ __forceinline__ int64_t ufrag_off(int s, int n, int nch, int V) { return ((int64_t)s * nch + n) * ufrag_v(V) * R; }
__device__ __forceinline__ int ufrag_idx(int c, int rt, int g, int l) { return (((c * 2 + rt) * 4 + g) * 64 + l) * 4; }
// Position of element (row r < 64, column v) in a fragment-order block.
__device__ __forceinline__ int ufrag_elem(int v, int r) {
  return ufrag_idx(v >> 5, r >> 5, (r >> 3) & 3, (v & 31) + 32 * ((r >> 2) & 1)) + (r & 3);
}
// Lane l's 16 accumulator values of strip c, row tile rt of one chunk's U
// block uc (zeros when the strip does not exist, c >= nstrip).
template <bool GUARD>
__device__ __forceinline__ void load_ufrag(float (&x)[16], const float* uc, int c, int nstrip, int rt, int l) {
  const bool ok = !GUARD || c < nstrip;
  const float* src = uc + ufrag_idx(ok ? c : 0, rt, 0, l);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float4 q = *reinterpret_cast<const float4*>(src + 256 * g);
    x[4 * g] = ok ? q.x : 0.f; x[4 * g + 1] = ok ? q.y : 0.f; x[4 * g + 2] = ok ? q.z : 0.f; x[4 * g + 3] = ok ? q.w : 0.f;
  }
}

// Per-chunk sizes (bf16 elements) of the MFMA fragment buffers.
__host__ __device__ __forceinline__ int frag_row_elems(int K, int per_lane) { return 2 * (K / 16) * 64 * per_lane; }
__host__ __device__ __forceinline__ int frag_col_elems(int K, int per_lane) { return ((K + 31) / 32) * 4 * 64 * per_lane; }

// Sum over the 16 lanes that share (lane / 16) within a wave.
__device__ __forceinline__ float sum16(float x) {
  x += __shfl_xor(x, 8, 16);
  x += __shfl_xor(x, 4, 16);
  x += __shfl_xor(x, 2, 16);
  x += __shfl_xor(x, 1, 16);
  return x;
}
__device__ __forceinline__ float sum64(float x) {
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
  return x;
}

// Load an R x KS slice (columns c0..c0+KS) of a saved [.., R, width] fp32 row
// block into LDS with optional per-row scale; zero past `width`.
__device__ __forceinline__ void stage_rows(float* dst, const float* src, int width, int c0,
                                           const float* row_scale) {
  for (int idx = threadIdx.x; idx < R * KS; idx += NT) {
    const int r = idx / KS, c = idx % KS;
    float x = (c0 + c < width) ? src[(int64_t)r * width + c0 + c] : 0.f;
    if (row_scale) x *= row_scale[r];
    dst[r * LDS_ + c] = x;
  }
}


// A struct in the kernel-argument segment copied word by word (scalar loads):
// the pack kernels read their entry this way (indexing a by-value argument
// would copy the whole argument to scratch).
template <typename T>
__device__ __forceinline__ void kernarg_copy(T& dst, const __attribute__((address_space(4))) T* src) {
  static_assert(sizeof(T) % 4 == 0, "word copy");
  const __attribute__((address_space(4))) uint32_t* s = (const __attribute__((address_space(4))) uint32_t*)src;
  uint32_t* d = reinterpret_cast<uint32_t*>(&dst);
#pragma unroll
  for (int i = 0; i < (int)(sizeof(T) / 4); ++i) d[i] = s[i];
}

// MFMA launchers for the bf16 state recurrences (gdn_state_mfma.hip); they
// return nonzero if the width is not built.
template <int KM>
int launch_state_fwd_mfma(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, int nch, hipStream_t st);
template <int KM>
int launch_state_bwd_mfma(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, const gpa_gdn_grads& gr, int nch,
                          hipStream_t st);
// Several problems of these kernels in one launch: workgroups wg0[i] ..
// wg0[i+1]-1 run problem i (mfma_state_workgroups(problem) of them).  `fast`
// when every problem has K == KM and V a multiple of 64; the backward's read
// gradient and state injections must be present in all problems or in none.
constexpr int GPA_MFMA_MAXP = 5;
struct MfmaPack {
  int n;
  int wg0[GPA_MFMA_MAXP], nvb[GPA_MFMA_MAXP], nch[GPA_MFMA_MAXP];
  gpa_gdn_problem p[GPA_MFMA_MAXP];
  gpa_gdn_saved sv[GPA_MFMA_MAXP];
  gpa_gdn_grads gr[GPA_MFMA_MAXP];
};
int mfma_state_workgroups(const gpa_gdn_problem& p);
template <int KM>
int launch_state_fwd_mfma_pack(const MfmaPack& pk, int total, bool fast, hipStream_t st);
template <int KM>
int launch_state_bwd_mfma_pack(const MfmaPack& pk, int total, bool fast, bool has_q, bool has_inj, hipStream_t st);
// MFMA chunk preparation (gdn_prep_mfma.hip); mf: write the bf16 fragments.
template <typename E, int KM>
int launch_prep_mfma(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, bool mf, int nch, hipStream_t st);
// bf16-MFMA output read and its chunk-local gradient (gdn_out_mfma.hip); bf16,
// kdim % 16 == 0 and vdim <= GPA_OUT_MFMA_MAX_V.
constexpr int GPA_OUT_MFMA_MAX_V = 256;
// The saved Qn and Kn rows hold bf16 (their values are exact in bf16: the
// model rounds them to the activation type) where only the bf16 MFMA out and
// dd0 kernels read them: bf16 problems with whole 16-wide key steps and V <=
// GPA_OUT_MFMA_MAX_V.  Elsewhere (the FMA kernels) they hold float.
__host__ __device__ inline bool qk_rows_bf16(const gpa_gdn_problem& p) {
  return p.dtype == GPA_DTYPE_BF16 && p.kdim % 16 == 0 && p.vdim <= GPA_OUT_MFMA_MAX_V;
}
template <int KM>
int launch_out_mfma(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, gpa_operand out, int nch, hipStream_t st);
template <int KM>
int launch_dd0_mfma(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, const gpa_gdn_grads& gr, int nch,
                    hipStream_t st);
// fp32-MFMA chunk backward (gdn_chunk_bwd_mfma.hip); needs kdim % 4 == 0.
template <typename E, int KM>
int launch_chunk_bwd_mfma(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, const gpa_gdn_grads& gr, int nch,
                          hipStream_t st);

}  // namespace gpa
