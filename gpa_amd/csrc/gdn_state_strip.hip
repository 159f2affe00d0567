// Sequential GDN state recurrences on bf16 MFMA, one 32-column strip of a
// stream's state per wave (gfx950).
//
// Per chunk n of a stream (reference src/gpa/ops.py:29-46, 80-85, chunked):
//   forward:  D = U - W S                     (64 x K) . (K x 32)
//             S = e^{G_C} S + Kn^T (diag(e^{G_C-G}) D)
//   backward: dD = dd0 + diag(e^{G_C-G}) (Kn dS)
//             dS = e^{G_C} dS + dstates[n] + Qn^T o - W^T dD
//
// Layout.  A wave holds its rows of a strip of S in MFMA accumulator tiles for
// the whole sequence and never shares them: both products of a chunk take S
// (or D) as their B operand straight from the accumulators.  An accumulator tile gives lane l rows 8g + 4(l/32) + 0..3
// (g < 4) of column l%32, whereas the B operand of v_mfma_f32_32x32x16_bf16
// wants rows 8(l/32) + 0..7 of a 16-row step; within each 16-row step the two
// lane halves hold each other's middle four rows, and one v_permlane32_swap
// per pair of registers exchanges them (swap_halves).  So the recurrence has
// no LDS round trip and no barrier between its two products.
//
// Work split.  NQ waves share a 32-column strip, each holding K/NQ of its K
// rows; the first product of a chunk is a sum over K, so each wave computes it
// over its own rows and the partial sums meet through LDS (one exchange and
// one barrier per chunk); the second product updates each wave's own rows.
// A workgroup of four waves covers 32 (4 / NQ) columns of one stream.  The
// forms: split (NQ = 2, 64 columns), quarter (NQ = 4, 32 columns; fewer rows
// per wave shorten the chunk step, which each wave's instruction stream
// bounds) and wide (NQ = 1, 128 columns, no exchange; for launches that would
// otherwise need more workgroups than the device has CUs).
//
// Operands.  The chunk's matrix fragments (W rows and Kn^T rows forward; Kn
// rows, W^T rows and Qn^T rows backward; the layouts of include/gpa_hip.h,
// written by gdn_prep) are the same for every strip of a stream: the
// workgroup copies them from global memory straight into LDS one chunk ahead
// (double-buffered, see dma_wave), and a barrier per chunk publishes them.
// Per-column data (U, D, dd0, o, injections, the saved states) goes between
// global memory and the wave's own registers, also one chunk ahead.
//
// Precision.  S, dS, D, dD, W and o are fp32 carried as bf16 hi + lo, each
// product keeping hi*hi + hi*lo + lo*hi; the normalised keys and queries are
// exact in bf16 (the reference rounds them to the activation type).
//
// Packing.  One launch runs up to GPA_STRIP_MAXP problems (scan groups) with
// the same key-width class: workgroup x belongs to the problem whose range of
// workgroups holds x.
#include <hip/hip_runtime.h>

#include "gdn_common.h"
#include "gdn_strip.h"
#include "mfma_tiles.h"

namespace gpa {
namespace {

constexpr int SW = 4;            // waves per workgroup
constexpr int SNT = 64 * SW;     // threads per workgroup
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // one 16-byte piece

struct BSplit {
  bf16x8 hi, lo;
};

// Exchange the upper-half lanes of x with the lower-half lanes of y.
__device__ __forceinline__ void swap_halves(uint32_t& x, uint32_t& y) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, y, false, false);
  x = r[0];
  y = r[1];
}

__device__ __forceinline__ bf16x8 as_b8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const uint4 u = make_uint4(a, b, c, d);
  bf16x8 r;
  __builtin_memcpy(&r, &u, 16);
  return r;
}

// Rows 16 hs .. 16 hs + 15 of a 32-row accumulator tile as the split B operand
// of one 16-deep MFMA step.
__device__ __forceinline__ BSplit acc_b(const f32x16& a, int hs) {
  uint2 XH, XL, YH, YL;
  bf2_split(a[8 * hs], a[8 * hs + 1], XH.x, XL.x);
  bf2_split(a[8 * hs + 2], a[8 * hs + 3], XH.y, XL.y);
  bf2_split(a[8 * hs + 4], a[8 * hs + 5], YH.x, YL.x);
  bf2_split(a[8 * hs + 6], a[8 * hs + 7], YH.y, YL.y);
  swap_halves(XH.x, YH.x);
  swap_halves(XH.y, YH.y);
  swap_halves(XL.x, YL.x);
  swap_halves(XL.y, YL.y);
  return BSplit{as_b8(XH.x, XH.y, YH.x, YH.y), as_b8(XL.x, XL.y, YL.x, YL.y)};
}

// Rows 16 ps + 8 (l/32) + 0..7 of column v of a value-major [V][64] fp32 block,
// split: the B operand of one 16-deep step read straight from memory.
template <bool GUARD>
__device__ __forceinline__ BSplit vc_b(const float* m, int v, int V, int ps, int l) {
  float x[8];
  const bool ok = !GUARD || v < V;
  const float* src = m + (int64_t)(ok ? v : 0) * R + 16 * ps + 8 * (l >> 5);
  const float4 a = *reinterpret_cast<const float4*>(src), c = *reinterpret_cast<const float4*>(src + 4);
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = c.x; x[5] = c.y; x[6] = c.z; x[7] = c.w;
  BSplit r;
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = ok ? x[e] : 0.f;
  split8(x, r.hi, r.lo);
  return r;
}

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Value-major [V][R] tile column v, rows row0 + 8g + 4(l/32) + 0..3, as the 16
// accumulator elements of lane l (zero for v >= V).  Loads use a clamped
// column so all four are in flight before any mask.
template <bool GUARD>
__device__ __forceinline__ void get_vc(float (&x)[16], const float* m, int v, int V, int row0, int l) {
  const float* src = m + (int64_t)(GUARD && v >= V ? 0 : v) * R + row0 + 4 * (l >> 5);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float4 q = *reinterpret_cast<const float4*>(src + 8 * g);
    const bool ok = !GUARD || v < V;
    x[4 * g] = ok ? q.x : 0.f; x[4 * g + 1] = ok ? q.y : 0.f; x[4 * g + 2] = ok ? q.z : 0.f; x[4 * g + 3] = ok ? q.w : 0.f;
  }
}

template <bool GUARD>
__device__ __forceinline__ void put_vc(float* m, int v, int V, int row0, const f32x16& x, int l) {
  if (GUARD && v >= V) return;
#pragma unroll
  for (int g = 0; g < 4; ++g)
    *reinterpret_cast<float4*>(m + (int64_t)v * R + row0 + 8 * g + 4 * (l >> 5)) =
        make_float4(x[4 * g], x[4 * g + 1], x[4 * g + 2], x[4 * g + 3]);
}

// Value-major [V][K] state: rows k0 + 8g + 4(l/32) + 0..3 of column v.
template <bool GUARD>
__device__ __forceinline__ void put_state(float* m, int v, int V, int K, int k0, const f32x16& x, int l) {
  if (GUARD && v >= V) return;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int k = k0 + 8 * g + 4 * (l >> 5);
    if (!GUARD || k < K)
      *reinterpret_cast<float4*>(m + (int64_t)v * K + k) = make_float4(x[4 * g], x[4 * g + 1], x[4 * g + 2], x[4 * g + 3]);
  }
}

template <bool GUARD>
__device__ __forceinline__ void get_state(f32x16& x, const float* m, int v, int V, int K, int k0, int l) {
  float t[16];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int k = k0 + 8 * g + 4 * (l >> 5);
    const bool ok = !GUARD || (v < V && k < K);
    const float4 q = *reinterpret_cast<const float4*>(m + (ok ? (int64_t)v * K + k : 0));
    t[4 * g] = ok ? q.x : 0.f; t[4 * g + 1] = ok ? q.y : 0.f; t[4 * g + 2] = ok ? q.z : 0.f; t[4 * g + 3] = ok ? q.w : 0.f;
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) x[r] = t[r];
}

// Key-major [K][V] state (initial state, final state and their gradients).
__device__ __forceinline__ void load_key_major(f32x16& x, const float* m, int64_t base, int v, int V, int K, int k0,
                                               int l) {
  if (!m) {
    x = f32x16{};
    return;
  }
  float t[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int k = k0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    t[r] = m[base + (k < K && v < V ? (int64_t)k * V + v : 0)];
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int k = k0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    x[r] = (k < K && v < V) ? t[r] : 0.f;
  }
}

__device__ __forceinline__ void store_key_major(float* m, int64_t base, int v, int V, int K, int k0, const f32x16& x,
                                                int l) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int k = k0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    if (k < K && v < V) m[base + (int64_t)k * V + v] = x[r];
  }
}

// The problem of a pack that workgroup x belongs to (the packs are short).  The
// pack is the kernel's only argument, so it sits at the start of the kernel
// argument segment: reading the entry through that pointer keeps the access a
// scalar load with a uniform offset (indexing the by-value argument makes the
// compiler copy the entry to scratch).
template <typename P, typename One>
__device__ __forceinline__ One pack_entry() {
  typedef const __attribute__((address_space(4))) P* KernargPtr;
  const KernargPtr pk = (KernargPtr)__builtin_amdgcn_kernarg_segment_ptr();
  int pi = 0;
#pragma unroll 1
  for (int i = 1; i < pk->n; ++i)
    if ((int)blockIdx.x >= pk->p[i].wg0) pi = i;
  One o;
  __builtin_memcpy(&o, (const __attribute__((address_space(4))) One*)&pk->p[pi], sizeof(One));
  return o;
}

// Chunk operands shared by the four waves go from global memory straight into
// LDS (global_load_lds_dwordx4: lane l of a wave writes 16 bytes at the LDS
// byte offset held in m0 plus 16 l), so they take no registers.  The
// instruction is issued from inline assembly so that the compiler neither
// reorders it nor adds waits for it; each wave drains its own copies with an
// explicit vmcnt(0) before the barrier that publishes them.  The kernels use
// m0 for nothing else.
__device__ __forceinline__ void dma_wave(const void* src_lane, uint32_t lds_byte) {
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_byte);  // wave-uniform by construction
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m0v), "v"(src_lane) : "memory", "m0");
}
// npieces (a multiple of 64) 16-byte pieces from src to LDS byte offset dst,
// 64 per wave-instruction, spread over the workgroup's waves.
__device__ __forceinline__ void dma_run(const u32x4* src, uint32_t dst, int npieces, int w, int l) {
  for (int j = w; j < npieces / 64; j += SW) dma_wave(src + j * 64 + l, dst + j * 1024);
}
// vmcnt(0), expcnt and lgkmcnt left at their maxima (gfx9 encoding), through
// the builtin so that the compiler knows every earlier load has completed.
__device__ __forceinline__ void dma_drain() { __builtin_amdgcn_s_waitcnt(0x0F70); }
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Gate factors of a chunk into LDS: f[r] = e^{G_C - G_r} for the 64 rows, then
// e^{G_C} (thread r < 64 of wave 0 computes row r).
__device__ __forceinline__ float gate_load(const float* gam, int tid) { return gam[tid & (R - 1)]; }
__device__ __forceinline__ void gate_store(float* gf, float g, int tid) {
  if (__builtin_amdgcn_readfirstlane(tid >> 6) == 0) {
    const float gc = __shfl(g, R - 1, 64);
    gf[tid] = __expf(gc - g);
    if (tid == 0) gf[R] = __expf(gc);
  }
}

constexpr int GATE_FLOATS = R + 4;

}  // namespace

// Both kernels.  Four waves: strip w / NQ of the workgroup's columns, part
// hk = w % NQ of the key rows (row tiles hk OT .. hk OT + OT - 1 of 32 rows,
// OT = KM / (32 NQ)).  LDS holds the chunk operands (double-buffered, except
// the backward's Kn rows), the gate factors (double-buffered) and one 64 x 32
// fp32 partial product per wave for the exchange.
// Per-wave slot of the exchange area (floats): a 64 x 32 fp32 partial product,
// or a wave's rows of its strip transposed for a store (RW rows + 4 of padding
// per column).
template <int NTW>
struct Slot {
  static constexpr int RW = 32 * NTW, LD = RW + 4;
  static constexpr int FLOATS = 32 * LD > 2048 ? 32 * LD : 2048;
  static constexpr int BYTES = SW * FLOATS * 4;
};

// Store the wave's NT row tiles (rows k0 .. k0 + 32 NT - 1) of its 32 columns
// (col0 ..) to a value-major [V][ld] block through its LDS slot, so that each
// global store instruction writes whole column runs (16 or 8 lanes per
// column) instead of one 16-byte piece of 64 different columns.
template <int NT, bool GUARD>
__device__ __forceinline__ void store_cols(float* slot, float* dst, int ld, int rows, int V, int col0, int k0,
                                           const f32x16 (&x)[NT], int l) {
  constexpr int RW = 32 * NT, LD = RW + 4, LPC = RW / 4, CPI = 64 / LPC;
#pragma unroll
  for (int i = 0; i < NT; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *reinterpret_cast<float4*>(slot + (l & 31) * LD + 32 * i + 8 * g + 4 * (l >> 5)) =
          make_float4(x[i][4 * g], x[i][4 * g + 1], x[i][4 * g + 2], x[i][4 * g + 3]);
#pragma unroll
  for (int it = 0; it < 32 / CPI; ++it) {
    const int c = it * CPI + l / LPC, r4 = (l % LPC) * 4, v = col0 + c, k = k0 + r4;
    const float4 y = *reinterpret_cast<const float4*>(slot + c * LD + r4);
    if (!GUARD || (v < V && k < rows)) *reinterpret_cast<float4*>(dst + (int64_t)v * ld + k) = y;
  }
}

// The reverse of store_cols: the wave's NT row tiles (rows k0 ..) of its 32
// columns from a value-major [V][ld] block, read as whole column runs into
// raw (cols_load), then put in the accumulator layout through the wave's LDS
// slot (cols_to_acc).
template <int NT>
struct ColsRaw {
  static constexpr int RW = 32 * NT, LPC = RW / 4, CPI = 64 / LPC, N = 32 / CPI;
  float4 x[N];
};
template <int NT, bool GUARD>
__device__ __forceinline__ void cols_load(ColsRaw<NT>& raw, const float* src, int ld, int rows, int V, int col0, int k0,
                                          int l) {
  using C = ColsRaw<NT>;
#pragma unroll
  for (int it = 0; it < C::N; ++it) {
    const int c = it * C::CPI + l / C::LPC, r4 = (l % C::LPC) * 4, v = col0 + c, k = k0 + r4;
    const bool ok = !GUARD || (v < V && k < rows);
    const float4 y = *reinterpret_cast<const float4*>(src + (ok ? (int64_t)v * ld + k : 0));
    raw.x[it] = ok ? y : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}
template <int NT>
__device__ __forceinline__ void cols_to_acc(f32x16 (&x)[NT], const ColsRaw<NT>& raw, float* slot, int l) {
  using C = ColsRaw<NT>;
  constexpr int LD = C::RW + 4;
#pragma unroll
  for (int it = 0; it < C::N; ++it)
    *reinterpret_cast<float4*>(slot + (it * C::CPI + l / C::LPC) * LD + (l % C::LPC) * 4) = raw.x[it];
#pragma unroll
  for (int i = 0; i < NT; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 q = *reinterpret_cast<const float4*>(slot + (l & 31) * LD + 32 * i + 8 * g + 4 * (l >> 5));
      x[i][4 * g] = q.x; x[i][4 * g + 1] = q.y; x[i][4 * g + 2] = q.z; x[i][4 * g + 3] = q.w;
    }
}

// A lane's 2 x 16 partial-product values into / out of the exchange area.
__device__ __forceinline__ void xch_put(float* x, const f32x16 (&d)[2], int l) {  // x: the wave's own slot
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *reinterpret_cast<float4*>(x + ((rt * 4 + g) * 64 + l) * 4) =
          make_float4(d[rt][4 * g], d[rt][4 * g + 1], d[rt][4 * g + 2], d[rt][4 * g + 3]);
}
__device__ __forceinline__ void xch_get(f32x16 (&d)[2], const float* x, int l) {  // x: the partner's slot
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 q = *reinterpret_cast<const float4*>(x + ((rt * 4 + g) * 64 + l) * 4);
      d[rt][4 * g] = q.x; d[rt][4 * g + 1] = q.y; d[rt][4 * g + 2] = q.z; d[rt][4 * g + 3] = q.w;
    }
}

// The full product of a strip from the NQ waves' parts: wave hk holds its own
// part in d, the others' parts are in their exchange slots (strip_slots +
// q slot_floats).  Summed in the order of the parts, ((p0 + p1) + p2) + p3, in
// every wave, so that every wave of a strip holds the same bits.
template <int NQ>
__device__ __forceinline__ void strip_sum(f32x16 (&sum)[2], const f32x16 (&d)[2], const float* strip_slots,
                                          int slot_floats, int hk, int l) {
  if constexpr (NQ == 1) {
    sum[0] = d[0];
    sum[1] = d[1];
  } else {
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) {
      f32x16 part[2];
      if (qi == hk) {
        part[0] = d[0];
        part[1] = d[1];
      } else {
        xch_get(part, strip_slots + qi * slot_floats, l);
      }
      if (qi == 0) {
        sum[0] = part[0];
        sum[1] = part[1];
      } else {
        sum[0] += part[0];
        sum[1] += part[1];
      }
    }
  }
}

template <int KM>
struct FwdLds {  // bytes
  static constexpr int WROW = 2 * (KM / 16) * 64 * 16 * 2, KCOL = (KM / 32) * 4 * 64 * 8 * 2;
  static constexpr int BUF = WROW + KCOL;
  static constexpr int GATE_OFF = 2 * BUF, XCH_OFF = GATE_OFF + 2 * GATE_FLOATS * 4;
  static constexpr int BYTES = XCH_OFF + Slot<KM / 64>::BYTES;
};
template <int KM, bool HAS_Q>
struct BwdLds {  // bytes
  static constexpr int KROW = 2 * (KM / 16) * 64 * 8 * 2, WCOL = (KM / 32) * 4 * 64 * 16 * 2;
  static constexpr int QCOL = HAS_Q ? (KM / 32) * 4 * 64 * 8 * 2 : 0;
  static constexpr int LATE = WCOL + QCOL;
  static constexpr int LATE_OFF = KROW, GATE_OFF = LATE_OFF + 2 * LATE, XCH_OFF = GATE_OFF + 2 * GATE_FLOATS * 4;
  static constexpr int BYTES = XCH_OFF + Slot<KM / 64>::BYTES;
};

// ---------------------------------------------------------------------------------------- forward
template <int KM, bool FAST, int NQ>
__global__ __launch_bounds__(SNT, 1) void gdn_state_fwd_strip(StripFwdPack pk) {
  static_assert(NQ == 2 || (FAST && KM == 128), "the wide and quarter forms are built for whole 128-key problems");
  constexpr int KT = KM / 32, K16M = KM / 16, NTW = KM / 64;
  constexpr int OT = KT / NQ;  // row tiles of S a wave owns
  constexpr int CPW = 32 * (SW / NQ);  // value columns per workgroup
  using L = FwdLds<KM>;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const StripFwdOne q = pack_entry<StripFwdPack, StripFwdOne>();
  const int local = blockIdx.x - q.wg0;
  const int s = local / q.wg_per_stream, cb = local % q.wg_per_stream;
  const int b = s / q.heads, h = s % q.heads;
  // Wave-uniform values are scalar: branches on them are scalar.
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, hk = w % NQ;
  const int K = FAST ? KM : q.K, V = q.V, nch = q.nch;
  const int K16 = K / 16, RB = (K + 31) / 32;
  const int wrow_n = 2 * K16 * 64 * 16, kcol_n = RB * 4 * 64 * 8;  // this problem's bf16 elements per chunk
  // Strip w/NQ of the workgroup's CPW columns, key part w%NQ (split: halves,
  // wide: all rows, quarter: quarters).
  const int col0 = CPW * cb + 32 * (w / NQ), v = col0 + (l & 31);
  const bool active = FAST || col0 < V;  // FAST: V % 64 == 0 (wide: V % 128 == 0)
  const uint32_t lds0 = lds_offset(smem_raw);
  auto wbuf = [&](int i) { return reinterpret_cast<const __bf16*>(smem_raw + i * L::BUF); };
  auto kbuf = [&](int i) { return reinterpret_cast<const __bf16*>(smem_raw + i * L::BUF + L::WROW); };
  float* gl0 = reinterpret_cast<float*>(smem_raw + L::GATE_OFF);
  float* slot = reinterpret_cast<float*>(smem_raw + L::XCH_OFF) + w * Slot<NTW>::FLOATS;
  const float* strip_slots = reinterpret_cast<const float*>(smem_raw + L::XCH_OFF) + (w - hk) * Slot<NTW>::FLOATS;

  const u32x4* wsrc = reinterpret_cast<const u32x4*>(q.wrow + (int64_t)s * nch * wrow_n);
  const u32x4* ksrc = reinterpret_cast<const u32x4*>(q.kcol + (int64_t)s * nch * kcol_n);
  const float* gsrc = q.gam + (int64_t)s * nch * R;
  auto fetch = [&](int n, int i) {  // chunk n's operands into buffer i
    dma_run(wsrc + (int64_t)n * (wrow_n / 8), lds0 + i * L::BUF, wrow_n / 8, w, l);
    dma_run(ksrc + (int64_t)n * (kcol_n / 8), lds0 + i * L::BUF + L::WROW, kcol_n / 8, w, l);
    return gate_load(gsrc + (int64_t)n * R, tid);
  };
  // The wave's rows of a strip go to a value-major block NTW row tiles at a
  // time (the capacity of its LDS slot).
  auto store_own = [&](float* dst, const f32x16 (&x)[OT]) {
    constexpr int SCH = OT < NTW ? OT : NTW;
#pragma unroll
    for (int h2 = 0; h2 < OT / SCH; ++h2) {
      f32x16 part[SCH];
#pragma unroll
      for (int i = 0; i < SCH; ++i) part[i] = x[h2 * SCH + i];
      store_cols<SCH, !FAST>(slot, dst, K, K, V, col0, 32 * (hk * OT + h2 * SCH), part, l);
    }
  };
  // Row tiles of D a wave saves: wide both, split and quarter the tile of its
  // index hk (quarter: waves 0 and 1 of a strip; saves_d).
  constexpr int DT = NQ == 1 ? 2 : 1;
  const bool saves_d = NQ != 4 || hk < 2;
  auto store_d = [&](float* dst, const f32x16 (&x)[DT]) {
    if (saves_d) store_cols<DT, !FAST>(slot, dst, R, R, V, col0, NQ == 1 ? 0 : 32 * hk, x, l);
  };

  f32x16 S[OT];
#pragma unroll
  for (int i = 0; i < OT; ++i)
    load_key_major(S[i], q.s0, (int64_t)b * q.s0_sb + (int64_t)h * q.s0_sh, v, V, K, 32 * (hk * OT + i), l);
  float g_next = fetch(0, 0);
  float ur[2][16], un[2][16];  // U of this chunk and of the next (fragment order, ufrag_idx)
  const int strip = col0 >> 5, nstrip = ufrag_v(V) >> 5;
  load_ufrag<!FAST>(ur[0], q.u + ufrag_off(s, 0, nch, V), strip, nstrip, 0, l);
  load_ufrag<!FAST>(ur[1], q.u + ufrag_off(s, 0, nch, V), strip, nstrip, 1, l);
  dma_drain();  // every load of the preamble: the loop then starts with none pending
  gate_store(gl0, g_next, tid);
  f32x16 dprev[DT] = {};  // this wave's row tiles of the previous chunk's D, stored one chunk late

  for (int n = 0; n < nch; ++n) {
    const int cur = n & 1;
    // The next chunk's operands into the other buffer (the last chunk fetches
    // itself again: the copies stay unconditional and are never read).
    const int nn = n + 1 < nch ? n + 1 : n;
    lds_barrier();
    // Every global access of the chunk is issued here, so that each has the
    // whole chunk step to complete before the drain at its end: the next
    // chunk's operands, gates and U, the previous chunk's D, this chunk's S.
    g_next = fetch(nn, cur ^ 1);
    f32x16 d[2] = {};
    if (active) {
      load_ufrag<!FAST>(un[0], q.u + ufrag_off(s, nn, nch, V), strip, nstrip, 0, l);
      load_ufrag<!FAST>(un[1], q.u + ufrag_off(s, nn, nch, V), strip, nstrip, 1, l);
      if (n > 0) store_d(q.delta + ((int64_t)s * nch + n - 1) * V * R, dprev);
      // (a) S_n -> the saved chunk-start states (own rows).
      store_own(q.states + ((int64_t)s * nch + n) * K * V, S);
      // (b) W S over the own rows, for both row tiles of W; every W fragment is
      // read from LDS before the first product.
      const __bf16* wf = wbuf(cur);
      bf16x8 wa[OT][2][2][2];  // [own tile][hs][rt][hi, lo]
#pragma unroll
      for (int i = 0; i < OT; ++i)
#pragma unroll
        for (int hs = 0; hs < 2; ++hs)
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            const int ks = 2 * (hk * OT + i) + hs;
            const __bf16* p = wf + (rt * K16 + (FAST || ks < K16 ? ks : 0)) * 1024 + l * 8;
            wa[i][hs][rt][0] = *reinterpret_cast<const bf16x8*>(p);
            wa[i][hs][rt][1] = *reinterpret_cast<const bf16x8*>(p + 512);
          }
#pragma unroll
      for (int i = 0; i < OT; ++i)
#pragma unroll
        for (int hs = 0; hs < 2; ++hs) {
          const int ks = 2 * (hk * OT + i) + hs;
          if (FAST || ks < K16) {
            const BSplit sb = acc_b(S[i], hs);
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
              d[rt] = mfma(wa[i][hs][rt][0], sb.hi, d[rt]);
              d[rt] = mfma(wa[i][hs][rt][0], sb.lo, d[rt]);
              d[rt] = mfma(wa[i][hs][rt][1], sb.hi, d[rt]);
            }
          }
        }
      if constexpr (NQ > 1) xch_put(slot, d, l);
    }
    // The waves of a strip meet here to exchange their parts of W S; a wide
    // wave holds the whole sum.
    if constexpr (NQ > 1) lds_barrier();
    if (active) {
      // (c) D = U - W S (split: own half + partner half, the same bits in both
      // waves since + commutes; half hk keeps row tile hk to save), then
      // scaled by e^{G_C - G}.
      f32x16 sum[2];
      strip_sum<NQ>(sum, d, strip_slots, Slot<NTW>::FLOATS, hk, l);
      const float* gf = gl0 + cur * GATE_FLOATS;
      const float decay = gf[R];
      f32x16 D[2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) D[rt][r] = ur[rt][r] - sum[rt][r];
        if constexpr (NQ == 1) dprev[rt] = D[rt];
        else if (rt == hk) dprev[0] = D[rt];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 f = *reinterpret_cast<const float4*>(gf + 32 * rt + 8 * g + 4 * (l >> 5));
          D[rt][4 * g] *= f.x; D[rt][4 * g + 1] *= f.y; D[rt][4 * g + 2] *= f.z; D[rt][4 * g + 3] *= f.w;
        }
      }
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int r = 0; r < 16; ++r) ur[rt][r] = un[rt][r];
      // (d) S = e^{G_C} S + Kn^T (e^{G_C-G} D) for the own rows.
      const __bf16* kf = kbuf(cur);
      bf16x8 ka[OT][4];
#pragma unroll
      for (int i = 0; i < OT; ++i)
#pragma unroll
        for (int ps = 0; ps < 4; ++ps) {
          const int t = hk * OT + i;
          ka[i][ps] = *reinterpret_cast<const bf16x8*>(kf + (((FAST || t < RB ? t : 0) * 4 + ps) * 64 + l) * 8);
        }
#pragma unroll
      for (int i = 0; i < OT; ++i) S[i] *= decay;
#pragma unroll
      for (int ps = 0; ps < 4; ++ps) {
        const BSplit db = acc_b(D[ps >> 1], ps & 1);
#pragma unroll
        for (int i = 0; i < OT; ++i) {
          const int t = hk * OT + i;
          if (FAST || t < RB) {
            S[i] = mfma(ka[i][ps], db.hi, S[i]);
            S[i] = mfma(ka[i][ps], db.lo, S[i]);
          }
        }
      }
    }
    gate_store(gl0 + (cur ^ 1) * GATE_FLOATS, g_next, tid);
    dma_drain();
  }
  if (active) {
    store_d(q.delta + ((int64_t)s * nch + nch - 1) * V * R, dprev);
#pragma unroll
    for (int i = 0; i < OT; ++i) {
      const int t = hk * OT + i;
      if (FAST || t < RB) store_key_major(q.final_state, (int64_t)s * K * V, v, V, K, 32 * t, S[i], l);
    }
  }
}

// --------------------------------------------------------------------------------------- backward
template <int KM, bool FAST, bool HAS_Q, bool HAS_INJ, int NQ>
__global__ __launch_bounds__(SNT, 1) void gdn_state_bwd_strip(StripBwdPack pk) {
  static_assert(NQ == 2 || (FAST && KM == 128), "the wide and quarter forms are built for whole 128-key problems");
  static_assert(NQ != 1 || !HAS_INJ, "the wide form is built without state injections");
  constexpr int KT = KM / 32, K16M = KM / 16, NTW = KM / 64;
  constexpr int OT = KT / NQ, DT = NQ == 1 ? 2 : 1;  // row tiles of dS a wave owns, of dD it saves
  constexpr int CPW = 32 * (SW / NQ);  // value columns per workgroup
  using L = BwdLds<KM, HAS_Q>;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const StripBwdOne q = pack_entry<StripBwdPack, StripBwdOne>();
  const int local = blockIdx.x - q.wg0;
  const int s = local / q.wg_per_stream, cb = local % q.wg_per_stream;
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, hk = w % NQ;
  const int K = FAST ? KM : q.K, V = q.V, nch = q.nch;
  const int K16 = K / 16, RB = (K + 31) / 32;
  const int krow_n = 2 * K16 * 64 * 8, wcol_n = RB * 4 * 64 * 16, qcol_n = HAS_Q ? RB * 4 * 64 * 8 : 0;
  // Strip w/NQ of the workgroup's CPW columns, key part w%NQ.
  const int col0 = CPW * cb + 32 * (w / NQ), v = col0 + (l & 31);
  const bool active = FAST || col0 < V;  // FAST: V % 64 == 0 (wide: V % 128 == 0)
  const uint32_t lds0 = lds_offset(smem_raw);
  const __bf16* kf = reinterpret_cast<const __bf16*>(smem_raw);  // Kn rows (one buffer)
  auto lbuf = [&](int i) { return reinterpret_cast<const __bf16*>(smem_raw + L::LATE_OFF + i * L::LATE); };
  float* gl0 = reinterpret_cast<float*>(smem_raw + L::GATE_OFF);
  float* slot = reinterpret_cast<float*>(smem_raw + L::XCH_OFF) + w * Slot<NTW>::FLOATS;
  const float* strip_slots = reinterpret_cast<const float*>(smem_raw + L::XCH_OFF) + (w - hk) * Slot<NTW>::FLOATS;

  const u32x4* ksrc = reinterpret_cast<const u32x4*>(q.krow + (int64_t)s * nch * krow_n);
  const u32x4* wsrc = reinterpret_cast<const u32x4*>(q.wcol + (int64_t)s * nch * wcol_n);
  const u32x4* qsrc = HAS_Q ? reinterpret_cast<const u32x4*>(q.qcol + (int64_t)s * nch * qcol_n) : wsrc;
  const float* gsrc = q.gam + (int64_t)s * nch * R;
  auto fetch_late = [&](int n, int i) {  // W^T and Qn^T rows of chunk n into late buffer i
    const uint32_t dst = lds0 + L::LATE_OFF + i * L::LATE;
    dma_run(wsrc + (int64_t)n * (wcol_n / 8), dst, wcol_n / 8, w, l);
    if (HAS_Q) dma_run(qsrc + (int64_t)n * (qcol_n / 8), dst + wcol_n * 2, qcol_n / 8, w, l);
    return gate_load(gsrc + (int64_t)n * R, tid);
  };
  auto fetch_early = [&](int n) { dma_run(ksrc + (int64_t)n * (krow_n / 8), lds0, krow_n / 8, w, l); };

  // The wave's rows of a strip go to a value-major block NTW row tiles at a
  // time (the capacity of its LDS slot).
  auto store_own = [&](float* dst, const f32x16 (&x)[OT]) {
    constexpr int SCH = OT < NTW ? OT : NTW;
#pragma unroll
    for (int h2 = 0; h2 < OT / SCH; ++h2) {
      f32x16 part[SCH];
#pragma unroll
      for (int i = 0; i < SCH; ++i) part[i] = x[h2 * SCH + i];
      store_cols<SCH, !FAST>(slot, dst, K, K, V, col0, 32 * (hk * OT + h2 * SCH), part, l);
    }
  };
  const bool saves_d = NQ != 4 || hk < 2;  // quarter: waves 0 and 1 of a strip save dD
  auto store_dd = [&](float* dst, const f32x16 (&x)[DT]) {
    if (saves_d) store_cols<DT, !FAST>(slot, dst, R, R, V, col0, NQ == 1 ? 0 : 32 * hk, x, l);
  };
  f32x16 dS[OT];
#pragma unroll
  for (int i = 0; i < OT; ++i)
    load_key_major(dS[i], q.dfinal, (int64_t)s * K * V, v, V, K, 32 * (hk * OT + i), l);
  float g_next = fetch_late(nch - 1, 0);
  fetch_early(nch - 1);
  // Per-column data of this chunk and of the next: dd0 and o (fragment order,
  // accumulator layout) with a read gradient; the state injection (value-major
  // [V][K], read as column runs and transposed when used) with one.
  const int strip = col0 >> 5, nstrip = ufrag_v(V) >> 5;
  float d0r[HAS_Q ? 2 : 1][16], d0n[HAS_Q ? 2 : 1][16];
  float orr[HAS_Q ? 2 : 1][16], onx[HAS_Q ? 2 : 1][16];
  ColsRaw<OT> inj, injn;
  auto load_cols = [&](int n, float (&d0)[HAS_Q ? 2 : 1][16], float (&ov)[HAS_Q ? 2 : 1][16], ColsRaw<OT>& ij) {
    if constexpr (HAS_Q) {
      load_ufrag<!FAST>(d0[0], q.dd0 + ufrag_off(s, n, nch, V), strip, nstrip, 0, l);
      load_ufrag<!FAST>(d0[1], q.dd0 + ufrag_off(s, n, nch, V), strip, nstrip, 1, l);
      load_ufrag<!FAST>(ov[0], q.o + ufrag_off(s, n, nch, V), strip, nstrip, 0, l);
      load_ufrag<!FAST>(ov[1], q.o + ufrag_off(s, n, nch, V), strip, nstrip, 1, l);
    }
    if constexpr (HAS_INJ)
      cols_load<OT, !FAST>(ij, q.dstates + ((int64_t)s * nch + n) * K * V, K, K, V, col0, 32 * OT * hk, l);
  };
  if (active) load_cols(nch - 1, d0r, orr, inj);
  dma_drain();  // every load of the preamble: the loop then starts with none pending
  gate_store(gl0, g_next, tid);
  f32x16 ddprev[DT] = {};  // this wave's row tiles of the previous (later) chunk's dD, stored one chunk late

  for (int n = nch - 1, it = 0; n >= 0; --n, ++it) {
    const int cur = it & 1;
    const int nn = n > 0 ? n - 1 : 0;  // the next (earlier) chunk; chunk 0 fetches itself again
    lds_barrier();
    // Every global access of the chunk is issued here (see the forward kernel).
    g_next = fetch_late(nn, cur ^ 1);
    f32x16 d[2] = {};
    const float* gf = gl0 + cur * GATE_FLOATS;
    const __bf16* lf = lbuf(cur);
    if (active) {
      load_cols(nn, d0n, onx, injn);
      if (n + 1 < nch) store_dd(q.ddelta + ((int64_t)s * nch + n + 1) * V * R, ddprev);
      // (a) dS at the end of chunk n -> dhend (own rows).
      store_own(q.dhend + ((int64_t)s * nch + n) * K * V, dS);
      // (b) B operands of the own rows of dS; Kn fragments from LDS.
      BSplit sb[OT][2];
#pragma unroll
      for (int i = 0; i < OT; ++i)
#pragma unroll
        for (int hs = 0; hs < 2; ++hs) sb[i][hs] = acc_b(dS[i], hs);
      bf16x8 ka[OT][2][2];  // [own tile][hs][rt]
#pragma unroll
      for (int i = 0; i < OT; ++i)
#pragma unroll
        for (int hs = 0; hs < 2; ++hs)
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            const int ks = 2 * (hk * OT + i) + hs;
            ka[i][hs][rt] = *reinterpret_cast<const bf16x8*>(kf + ((rt * K16 + (FAST || ks < K16 ? ks : 0)) * 64 + l) * 8);
          }
      // (c) the update terms that do not need dD: e^{G_C} dS + dstates[n] + Qn^T o,
      // interleaved with Kn dS over the own rows.
      const float decay = gf[R];
      f32x16 ij[OT];
      if constexpr (HAS_INJ) cols_to_acc(ij, inj, slot, l);
#pragma unroll
      for (int i = 0; i < OT; ++i) {
        dS[i] *= decay;
        if constexpr (HAS_INJ) dS[i] += ij[i];
      }
      BSplit ob[HAS_Q ? 4 : 1];  // o as the B operand of the four position steps
      if constexpr (HAS_Q) {
#pragma unroll
        for (int ps = 0; ps < 4; ++ps) {
          f32x16 ot;
#pragma unroll
          for (int r = 0; r < 16; ++r) ot[r] = orr[ps >> 1][r];
          ob[ps] = acc_b(ot, ps & 1);
        }
      }
#pragma unroll
      for (int i = 0; i < OT; ++i)
#pragma unroll
        for (int hs = 0; hs < 2; ++hs) {
          const int ks = 2 * (hk * OT + i) + hs;
          if (FAST || ks < K16) {
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
              d[rt] = mfma(ka[i][hs][rt], sb[i][hs].hi, d[rt]);
              d[rt] = mfma(ka[i][hs][rt], sb[i][hs].lo, d[rt]);
            }
          }
          if constexpr (HAS_Q) {
            const int t = hk * OT + i;
            if (FAST || t < RB) {
#pragma unroll
              for (int pp = 0; pp < 2; ++pp) {
                const int ps = 2 * hs + pp;
                const bf16x8 qq = *reinterpret_cast<const bf16x8*>(lf + wcol_n + ((t * 4 + ps) * 64 + l) * 8);
                dS[i] = mfma(qq, ob[ps].hi, dS[i]);
                dS[i] = mfma(qq, ob[ps].lo, dS[i]);
              }
            }
          }
        }
      if constexpr (NQ > 1) xch_put(slot, d, l);
    }
    // The waves of a strip exchange their parts of Kn dS here; every wave has read
    // this chunk's Kn rows before the copy of the next chunk's overwrites them.
    lds_barrier();
    fetch_early(nn);  // Kn rows are read only before the barrier above
    if (active) {
      // (d) dD = dd0 + e^{G_C-G} (half 0 + half 1) (saved: half hk stores row
      // tile hk), negated.
      f32x16 sum[2];
      strip_sum<NQ>(sum, d, strip_slots, Slot<NTW>::FLOATS, hk, l);
      f32x16 nd[2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        f32x16 dd;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 f = *reinterpret_cast<const float4*>(gf + 32 * rt + 8 * g + 4 * (l >> 5));
          const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r = 4 * g + j;
            dd[r] = (HAS_Q ? d0r[rt][r] : 0.f) + fv[j] * sum[rt][r];
          }
        }
        if constexpr (NQ == 1) ddprev[rt] = dd;
        else if (rt == hk) ddprev[0] = dd;
        nd[rt] = -dd;
      }
      if constexpr (HAS_Q) {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            d0r[rt][r] = d0n[rt][r];
            orr[rt][r] = onx[rt][r];
          }
      }
      if constexpr (HAS_INJ) inj = injn;
      // (e) dS += W^T (-dD) for the own rows.
      bf16x8 wa[OT][4][2];  // [own tile][ps][hi, lo]
#pragma unroll
      for (int i = 0; i < OT; ++i)
#pragma unroll
        for (int ps = 0; ps < 4; ++ps) {
          const int t = hk * OT + i;
          const __bf16* p = lf + ((FAST || t < RB ? t : 0) * 4 + ps) * 1024 + l * 8;
          wa[i][ps][0] = *reinterpret_cast<const bf16x8*>(p);
          wa[i][ps][1] = *reinterpret_cast<const bf16x8*>(p + 512);
        }
#pragma unroll
      for (int ps = 0; ps < 4; ++ps) {
        const BSplit db = acc_b(nd[ps >> 1], ps & 1);
#pragma unroll
        for (int i = 0; i < OT; ++i) {
          const int t = hk * OT + i;
          if (FAST || t < RB) {
            dS[i] = mfma(wa[i][ps][0], db.hi, dS[i]);
            dS[i] = mfma(wa[i][ps][0], db.lo, dS[i]);
            dS[i] = mfma(wa[i][ps][1], db.hi, dS[i]);
          }
        }
      }
    }
    gate_store(gl0 + (cur ^ 1) * GATE_FLOATS, g_next, tid);
    dma_drain();
  }
  if (active) {
    store_dd(q.ddelta + (int64_t)s * nch * V * R, ddprev);
#pragma unroll
    for (int i = 0; i < OT; ++i) {
      const int t = hk * OT + i;
      if (FAST || t < RB) store_key_major(q.ds0, (int64_t)s * K * V, v, V, K, 32 * t, dS[i], l);
    }
  }
}

// ---------------------------------------------------------------------------------------- launch
namespace {

template <typename F>
int allow_lds_strip(F kernel, size_t bytes) {
  if (bytes <= 65536) return GPA_HIP_OK;
  const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  return err == hipSuccess ? GPA_HIP_OK : fail(GPA_HIP_EHIP, "hipFuncSetAttribute(max dynamic LDS) failed");
}

}  // namespace

int strip_wg_per_stream(int vdim, int nq) {
  const int cols = 32 * (SW / nq);
  return (vdim + cols - 1) / cols;
}

StripFwdOne strip_fwd_one(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, int nch, int wg0, int nq) {
  StripFwdOne o{};
  o.K = p.kdim;
  o.V = p.vdim;
  o.heads = p.heads;
  o.nch = nch;
  o.wg0 = wg0;
  o.wg_per_stream = strip_wg_per_stream(p.vdim, nq);
  o.s0 = p.s0;
  o.s0_sb = p.s0_sb;
  o.s0_sh = p.s0_sh;
  o.wrow = static_cast<const __bf16*>(sv.wrow);
  o.kcol = static_cast<const __bf16*>(sv.kcol);
  o.u = sv.u;
  o.gam = sv.gam;
  o.delta = sv.delta;
  o.states = sv.states;
  o.final_state = sv.final;
  return o;
}

StripBwdOne strip_bwd_one(const gpa_gdn_problem& p, const gpa_gdn_saved& sv, const gpa_gdn_grads& gr, int nch,
                          int wg0, bool has_q, int nq) {
  StripBwdOne o{};
  o.K = p.kdim;
  o.V = p.vdim;
  o.heads = p.heads;
  o.nch = nch;
  o.wg0 = wg0;
  o.wg_per_stream = strip_wg_per_stream(p.vdim, nq);
  o.dfinal = gr.dfinal;
  o.dstates = gr.dstates;
  o.dd0 = has_q ? gr.dd0 : nullptr;
  o.o = has_q ? gr.o : nullptr;
  o.ddelta = gr.ddelta;
  o.dhend = gr.dhend;
  o.ds0 = gr.ds0;
  o.krow = static_cast<const __bf16*>(sv.krow);
  o.wcol = static_cast<const __bf16*>(sv.wcol);
  o.qcol = has_q ? static_cast<const __bf16*>(sv.qcol) : nullptr;
  o.gam = sv.gam;
  return o;
}

template <int KM, bool FAST, int NQ>
int launch_fwd_strip(const StripFwdPack& pk, int total_wg, hipStream_t st) {
  const size_t lds = FwdLds<KM>::BYTES;
  if (int rc = allow_lds_strip(gdn_state_fwd_strip<KM, FAST, NQ>, lds)) return rc;
  hipLaunchKernelGGL((gdn_state_fwd_strip<KM, FAST, NQ>), dim3(total_wg), dim3(SNT), lds, st, pk);
  return GPA_HIP_OK;
}

template <int KM>
int launch_state_fwd_strip(const StripFwdPack& pk, int total_wg, bool fast, int nq, hipStream_t st) {
  if constexpr (KM == 128) {
    if (nq == 1 && fast) return launch_fwd_strip<KM, true, 1>(pk, total_wg, st);
    if (nq == 4 && fast) return launch_fwd_strip<KM, true, 4>(pk, total_wg, st);
  }
  if (nq != 2) return fail(GPA_HIP_EINVAL, "strip forward: the wide and quarter forms are built for whole 128-key groups");
  return fast ? launch_fwd_strip<KM, true, 2>(pk, total_wg, st) : launch_fwd_strip<KM, false, 2>(pk, total_wg, st);
}

template <int KM, bool FAST, bool HAS_Q, bool HAS_INJ, int NQ = 2>
int launch_bwd_strip(const StripBwdPack& pk, int total_wg, hipStream_t st) {
  const size_t lds = BwdLds<KM, HAS_Q>::BYTES;
  if (int rc = allow_lds_strip(gdn_state_bwd_strip<KM, FAST, HAS_Q, HAS_INJ, NQ>, lds)) return rc;
  hipLaunchKernelGGL((gdn_state_bwd_strip<KM, FAST, HAS_Q, HAS_INJ, NQ>), dim3(total_wg), dim3(SNT), lds, st, pk);
  return GPA_HIP_OK;
}

template <int KM>
int launch_state_bwd_strip(const StripBwdPack& pk, int total_wg, bool fast, bool has_q, bool has_inj, int nq,
                           hipStream_t st) {
  if constexpr (KM == 128) {
    if (nq == 1 && fast && !has_inj)
      return has_q ? launch_bwd_strip<KM, true, true, false, 1>(pk, total_wg, st)
                   : launch_bwd_strip<KM, true, false, false, 1>(pk, total_wg, st);
    if (nq == 4 && fast) {
      if (has_q) return has_inj ? launch_bwd_strip<KM, true, true, true, 4>(pk, total_wg, st)
                                : launch_bwd_strip<KM, true, true, false, 4>(pk, total_wg, st);
      return has_inj ? launch_bwd_strip<KM, true, false, true, 4>(pk, total_wg, st)
                     : launch_bwd_strip<KM, true, false, false, 4>(pk, total_wg, st);
    }
  }
  if (nq != 2)
    return fail(GPA_HIP_EINVAL, "strip backward: the wide form (no injections) and the quarter form are built for "
                                "whole 128-key groups");
  if (fast) {
    if (has_q) return has_inj ? launch_bwd_strip<KM, true, true, true>(pk, total_wg, st)
                              : launch_bwd_strip<KM, true, true, false>(pk, total_wg, st);
    return has_inj ? launch_bwd_strip<KM, true, false, true>(pk, total_wg, st)
                   : launch_bwd_strip<KM, true, false, false>(pk, total_wg, st);
  }
  if (has_q) return has_inj ? launch_bwd_strip<KM, false, true, true>(pk, total_wg, st)
                            : launch_bwd_strip<KM, false, true, false>(pk, total_wg, st);
  return has_inj ? launch_bwd_strip<KM, false, false, true>(pk, total_wg, st)
                 : launch_bwd_strip<KM, false, false, false>(pk, total_wg, st);
}

template int launch_state_fwd_strip<64>(const StripFwdPack&, int, bool, int, hipStream_t);
template int launch_state_fwd_strip<128>(const StripFwdPack&, int, bool, int, hipStream_t);
template int launch_state_bwd_strip<64>(const StripBwdPack&, int, bool, bool, bool, int, hipStream_t);
template int launch_state_bwd_strip<128>(const StripBwdPack&, int, bool, bool, bool, int, hipStream_t);

}  // namespace gpa
