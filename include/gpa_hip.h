/*
 * gpa_hip.h -- C ABI of libgpa_hip.so, the gfx950 HIP backend of the DenseGPA
 * attention core.
 *
 * Every entry point takes plain device pointers, sizes and element strides,
 * enqueues its kernels on the given HIP stream and returns 0 on success or a
 * negative GPA_HIP_E* code; gpa_hip_last_error() then describes the failure
 * (per calling thread).  The library never allocates device memory, never
 * synchronises and keeps no mutable global state: every buffer (inputs,
 * outputs, the intermediates a backward pass needs) is owned by the caller,
 * so calls are reentrant and may be captured into a HIP graph.
 *
 * Operand convention.  A scan runs `batch*heads` independent streams.  Element
 * (stream s = b*heads + h, token t, feature d) of a gpa_operand lives at
 * ptr[b*sb + t*st + h*sh + d]: this addresses the reference's time-first
 * [B,T,H,D] tensors (and any packed or expanded view of them) without copies.
 * Per-token scalars (g, beta, their gradients) use the same rule with d = 0.
 *
 * Chunk geometry.  Position p of a stream holds token t = p - offset; the
 * positions before token 0 and after token T-1 are "void" (no state change, no
 * output).  Chunk n covers positions [n*chunk, (n+1)*chunk) and is stored as
 * GPA_CHUNK_ROWS rows, the rows past `chunk` also void.  nchunks =
 * ceil((offset + tokens) / chunk).  Chunk boundaries are the block boundaries
 * of the block-lagged model (reference src/gpa/attention.py:397).
 */
#ifndef GPA_HIP_H
#define GPA_HIP_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GPA_HIP_ABI_VERSION 4
#define GPA_CHUNK_ROWS 64   /* rows per stored chunk; chunk <= 64 */
#define GPA_MAX_KDIM 256    /* key width of a scan (the reduced dimension) */
#define GPA_MAX_VDIM 1024   /* value width of a scan */

#define GPA_HIP_OK 0
#define GPA_HIP_EINVAL (-1)      /* bad argument: shape, pointer, stride */
#define GPA_HIP_EUNSUPPORTED (-2) /* valid but not built: dtype, width */
#define GPA_HIP_EHIP (-3)        /* a HIP runtime call failed */

#define GPA_DTYPE_F32 0
#define GPA_DTYPE_BF16 1

typedef struct gpa_operand {
    void *ptr;
    int64_t sb, st, sh;
} gpa_operand;

/* One group of GDN scans with common widths (reference ops.py:49-85 and the
 * packed level/edge launches of packed.py:77,121,155). */
typedef struct gpa_gdn_problem {
    int32_t batch, heads;   /* streams = batch*heads */
    int32_t tokens;         /* T >= 1 real tokens */
    int32_t offset;         /* void positions before token 0, 0 <= offset < chunk */
    int32_t chunk;          /* 1..GPA_CHUNK_ROWS */
    int32_t kdim, vdim;     /* 1..GPA_MAX_KDIM, 1..GPA_MAX_VDIM */
    int32_t dtype;          /* GPA_DTYPE_*: q, k, v, out, dout element type */
    gpa_operand q, k, v;    /* q.ptr may be NULL: no output read */
    gpa_operand g, beta;    /* float32 log-decay (<= 0) and write strength */
    const float *s0;        /* [batch,heads,K,V] at s0[b*s0_sb + h*s0_sh + k*V + v]; NULL = zeros */
    int64_t s0_sb, s0_sh;
} gpa_gdn_problem;

/* Caller-owned intermediates, stream-major and contiguous (S = streams,
 * N = nchunks, per chunk):
 *   kn, qn         f32 [S,N,64,K]   normalised keys / queries (rows = positions)
 *   w              f32 [S,N,64,K]   W = T diag(b e^G) Kn  (FMA path only)
 *   u, delta       f32 [S,N,V,64]   U = T diag(b) V, D = U - W S_n  (value-major)
 *   tri            f32 [S,N,64,64]  T = (I + A)^-1
 *   gam, beta      f32 [S,N,64]     in-chunk cumulative log decay, beta (void rows 0)
 *   states         f32 [S,N,V,K]    state at the start of every chunk, value-major
 *                                   (element (k,v) of chunk n at [v*K + k])
 *   final          f32 [S,K,V]      state after the last token (key-major)
 * On the MFMA path (gpa_gdn_path() == 1) the sequential kernels read their
 * matrix operands as bf16 MFMA fragments written by the chunk kernel; with
 * K16 = K/16 and RB = ceil(K/32), per chunk:
 *   wrow  [2][K16][64][16]  W rows:     lane l of fragment (rt,ks) holds
 *                           W[32rt + l%32][16ks + 8(l/32) + e], e<8, as hi then lo
 *   wcol  [RB][4][64][16]   W^T rows:   fragment (rb,cs), lane l, element e is
 *                           W[16cs + 8(l/32) + e][32rb + l%32], hi then lo
 *   krow  [2][K16][64][8]   Kn rows (exact in bf16), same placement as wrow
 *   kcol  [RB][4][64][8]    Kn^T rows, same placement as wcol
 *   qcol  [RB][4][64][8]    Qn^T rows (only with a query)
 * qn is written only when problem.q.ptr != NULL. */
typedef struct gpa_gdn_saved {
    float *kn, *qn, *w, *u, *delta, *tri, *gam, *beta, *states, *final;
    void *wrow, *wcol, *krow, *kcol, *qcol;
} gpa_gdn_saved;

/* Backward inputs and outputs.  dout (problem dtype, strided like out) may be
 * NULL (no read gradient); dstates f32 [S,N,V,K] (value-major, like states)
 * injects gradients of the chunk-start states (NULL = none); dfinal f32
 * [S,K,V] (NULL = none).  Caller-owned f32 scratch: dd0, o, ddelta
 * [S,N,V,64], dhend [S,N,V,K], dw [S,N,64,K].  Gradient outputs are f32
 * operands: dq (skipped when q was NULL), dk [.. K], dv [.. V], dg, dbeta per
 * token; ds0 [S,K,V] contiguous. */
typedef struct gpa_gdn_grads {
    gpa_operand dout;
    const float *dstates, *dfinal;
    float *dd0, *o, *ddelta, *dhend, *dw;
    gpa_operand dq, dk, dv, dg, dbeta;
    float *ds0;
} gpa_gdn_grads;

/* Optional kernel timing: when non-NULL, events[i] is recorded on the stream
 * before the i-th kernel an entry point launches and events[n] after the
 * last one (n = *launched on return, at most GPA_MAX_TIMED).  The events are
 * created and read by the caller (hipEventCreate / hipEventElapsedTime). */
#define GPA_MAX_TIMED 4
typedef struct gpa_timing {
    hipEvent_t events[GPA_MAX_TIMED + 1];
    int32_t launched;
} gpa_timing;

int gpa_hip_abi_version(void);
const char *gpa_hip_last_error(void);
/* Number of chunks a problem spans (0 on invalid geometry). */
int32_t gpa_gdn_nchunks(int32_t tokens, int32_t offset, int32_t chunk);
/* 1 when the problem runs its state recurrences on bf16 MFMA (bf16 data,
 * K a multiple of 16) and needs the fragment buffers; 0 on the fp32 FMA path. */
int32_t gpa_gdn_path(const gpa_gdn_problem *problem);

/* Forward chunked gated-delta-rule scan; `out` (problem dtype) receives
 * u(q_t)^T S_t when q.ptr != NULL.
 * Replaces reference src/gpa/ops.py:49-85 (gdn_scan, backend dispatch at
 * ops.py:58-79) for a whole group of streams. */
int gpa_gdn_forward(const gpa_gdn_problem *problem, const gpa_gdn_saved *saved,
                    gpa_operand out, gpa_timing *timing, hipStream_t stream);

/* Backward of gpa_gdn_forward from its saved intermediates (the autograd of
 * ops.py:49-85 in the reference, plus chunk-start state injections). */
int gpa_gdn_backward(const gpa_gdn_problem *problem, const gpa_gdn_saved *saved,
                     const gpa_gdn_grads *grads, gpa_timing *timing, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Batched single-token decode step of the whole DenseGPA core (the reference's
 * chunk-mode decode: _block_segment at T = 1, src/gpa/attention.py:299-345 and
 * 396-405), default flags: positional_mode gated or none, linear slot
 * features, no control input, legacy route reader, no rsa/product/shared
 * centre/balanced bridge/learned read scale.  One workgroup per (b, h) stream
 * walks levels, edges, route reader and outer reads for the token; every state
 * matrix is read and written once.
 *
 * States are fp32, [B, H, rows, cols] with each head's matrix contiguous and a
 * batch stride `sb` in elements (0 for a prefix broadcast over the batch).
 * Outputs are new, contiguous [B, H, rows, cols] buffers (inputs are never
 * written).  snap_inner/snap_outer are the block-start snapshots the write and
 * the residuals read (the current states when the token starts a block).
 * Parameters are the module's fp32 tensors, contiguous, in the shapes of
 * src/gpa/attention.py:95-142. */
#define GPA_DECODE_MAX_LEVELS 4
#define GPA_DECODE_MAX_EDGES 12
#define GPA_DECODE_MAX_WIDTH 256  /* key_dim, value_dim and every slot count */

typedef struct gpa_decode_state {
    const float *ptr;
    int64_t sb;
} gpa_decode_state;

typedef struct gpa_decode_level {
    int32_t slots;
    const float *center, *gate_weight, *gate_bias;            /* [H,M,Dk], [H,Dk,4], [H,4] */
    const float *route_weight, *query_weight;                 /* [H,M,M], [H,Dk,M] */
    const float *route_up, *route_down;                       /* [H,M,2M], [H,2M,M] */
    gpa_decode_state inner, outer, count;                     /* [B,H,Dk,M], [B,H,M,Dv], [B,H,M] */
    gpa_decode_state snap_inner, snap_outer;                  /* frozen [B,H,Dk,M], [B,H,M,Dv] */
    float *inner_out, *outer_out, *count_out;
} gpa_decode_level;

typedef struct gpa_decode_problem {
    int32_t batch, heads, key_dim, value_dim, levels, dtype;
    int32_t positional_none;        /* 1: decay gates are zero (positional_mode "none") */
    float read_scale, query_scale, beta_max;
    gpa_operand q, k, v, out;       /* [B,1,H,D] activations (t stride unused) */
    const float *residual_raw;      /* [L,H,2] */
    const float *count_gain_raw, *route_mlp_gain, *output_logits, *relation_gain;  /* [L,H] */
    const float *edge_logits, *relation_decay_raw, *relation_beta_raw;            /* [E,H] */
    gpa_decode_level level[GPA_DECODE_MAX_LEVELS];
    gpa_decode_state relation[GPA_DECODE_MAX_EDGES];   /* edge e = (i -> j), i-major: [B,H,Mi,Mj] */
    float *relation_out[GPA_DECODE_MAX_EDGES];
} gpa_decode_problem;

/* One decode token of every stream (no autograd).  Replaces the T = 1 call of
 * DenseGPA.forward in chunk mode (reference attention.py:347-413). */
int gpa_decode_step(const gpa_decode_problem *problem, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* GPA_HIP_H */
