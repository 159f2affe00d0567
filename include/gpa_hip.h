/*
 * gpa_hip.h -- C ABI of libgpa_hip.so, the gfx950 HIP backend of the DenseGPA
 * attention core.
 *
 * Every entry point takes plain device pointers, sizes and element strides,
 * enqueues its kernels on the given HIP stream and returns 0 on success or a
 * negative GPA_HIP_E* code; gpa_hip_last_error() then describes the failure
 * (per calling thread).  The library never allocates device memory and never
 * synchronises: every buffer (inputs, outputs, the intermediates a backward
 * pass needs) is owned by the caller, so calls are reentrant and may be
 * captured into a HIP graph.  Library-held state, all of it per device:
 *  - gpa_gdn_forward_many / gpa_gdn_backward_many keep one side stream and
 *    two events per device, created (default priority, hipStreamNonBlocking)
 *    on the first call that needs them and kept for the process.  When a
 *    call mixes 256-key groups with narrower ones (or, forward and backward,
 *    packs two or more strip groups), part of its groups run on that stream:
 *    the call records a fork event on the caller's stream, makes the side
 *    stream wait for it, enqueues, and makes the caller's stream wait for a
 *    join event on every return path, so later work on the caller's stream
 *    is ordered after all of the call's kernels.  The enqueue sequence runs
 *    under a process-wide mutex.  Calls under graph capture and timed calls
 *    never take the side stream (they stay on the caller's stream).
 *  - gpa_gdn_scan_noalloc keeps its intermediates in a static per-device
 *    array (see there).
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

#define GPA_HIP_ABI_VERSION 31
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
 *   kn, qn         f32 [S,N,64,K]   normalised keys / queries (rows = positions); for bf16
 *                                   problems with K % 16 == 0 and V <= 256, qn holds its
 *                                   exact bf16 values instead (bf16 [S,N,64,K] in the first
 *                                   half of the buffer) and kn is not written (the krow
 *                                   fragments below carry the same values)
 *   w              f32 [S,N,64,K]   W = T diag(b e^G) Kn  (FMA path only)
 *   u, delta       f32 [S,N,V,64]   U = T diag(b) V, D = U - W S_n  (value-major; on the
 *                                   MFMA path u is in fragment order instead, per chunk
 *                                   [ceil(V/32)][2][4][64][4]: strip c, row tile rt, group
 *                                   g, lane l holds U rows 32rt + 8g + 4(l/32) + 0..3 of
 *                                   column 32c + l%32, zero past V)
 *   tri            f32 [S,N,64,64]  T = (I + A)^-1
 *   gam, beta      f32 [S,N,64]     in-chunk cumulative log decay, beta (void rows 0)
 *   states         f32 [S,N,V,K]    state at the start of every chunk, value-major
 *                                   (element (k,v) of chunk n at [v*K + k])
 *   final          f32 [S,K,V]      state after the last token (key-major)
 * On the MFMA path (gpa_gdn_path() == 1) the sequential kernels read their
 * matrix operands as bf16 MFMA fragments written by the chunk kernel; with
 * K16 = K/16 and RB = ceil(K/32), per chunk:
 *   wrow  [2][K16][2][64][8] W rows:    lane l of fragment (rt,ks) holds
 *                           W[32rt + l%32][16ks + 8(l/32) + e], e<8, split
 *                           into bf16 hi (plane 0) and lo = x - hi (plane 1)
 *   wcol  [RB][4][2][64][8]  W^T rows:   fragment (rb,cs), lane l, element e is
 *                           W[16cs + 8(l/32) + e][32rb + l%32], hi / lo planes
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
 * [S,N,V,64], dhend [S,N,V,K], dw [S,N,64,K]; on the MFMA path dd0 and o are
 * in the fragment order of u (ceil(V/32) whole strips per chunk).  Gradient outputs: dq
 * (skipped when q was NULL), dk [.. K], dv [.. V] in the problem dtype
 * (rounded once from fp32); dg, dbeta f32 per token; ds0 [S,K,V] f32
 * contiguous. */
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
#define GPA_MAX_TIMED 40
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

/* Forward / backward of up to GPA_GDN_MAX_PACK independent scan groups in one
 * call (saved[i], outs[i], grads[i] belong to problems[i]): the packed level
 * and edge launches of the reference (packed.py:77, 121, 155 pack the levels
 * or the edges into one scan over L*H or E*H heads; staged.py:14-35 pairs the
 * A and B scans of a level).  The chunk-parallel kernels run once per group;
 * the sequential state recurrences of all groups on the bf16 strip kernels
 * (K <= 128) advance together in one launch per key-width class (and, in the
 * backward, per presence of a read gradient and of state injections).
 * Results are those of one gpa_gdn_forward / gpa_gdn_backward per group, up
 * to the order of the sums over the key rows when a strip launch exceeds the
 * device's compute units and runs in its wide form (one workgroup per 128
 * value columns); the groups must not write a buffer another one reads.  timing (may be NULL)
 * marks every launch in order: the preps, the state launches, the reads
 * (forward); the dd0 kernels, the state launches, the chunk kernels
 * (backward). */
#define GPA_GDN_MAX_PACK 12
int gpa_gdn_forward_many(const gpa_gdn_problem *problems, const gpa_gdn_saved *saved, const gpa_operand *outs,
                         int32_t n, gpa_timing *timing, hipStream_t stream);
int gpa_gdn_backward_many(const gpa_gdn_problem *problems, const gpa_gdn_saved *saved,
                          const gpa_gdn_grads *grads, int32_t n, gpa_timing *timing, hipStream_t stream);

/* A late read: `out` = u(q_t)^T S_t for a query that arrives after the scan.
 * `saved` holds the intermediates of a gpa_gdn_forward that ran with
 * problem.q = NULL (same k, v, g, beta, s0, chunk, offset); this call fills
 * saved.qn and saved.qcol for the new query (problem.q) and runs the read.
 * The result equals gpa_gdn_forward with that query, without repeating the
 * state recurrence.  Needs bf16, K a multiple of 16 up to 256, V a multiple
 * of 8 up to 256.  Replaces the second pass of the same recurrence that the
 * reference makes for a level's outer read (src/gpa/attention.py:333-341
 * reads the B memory that :318-329 updates). */
int gpa_gdn_read(const gpa_gdn_problem *problem, const gpa_gdn_saved *saved, gpa_operand out,
                 hipStream_t stream);

/* The query gradient of a late read alone: dq (f32 operand, [B,T,H,K]) from
 * dout.  The read's other gradients are those of gpa_gdn_backward with the
 * same problem (query set), saved (qn, qcol filled) and dout. */
int gpa_gdn_read_backward(const gpa_gdn_problem *problem, const gpa_gdn_saved *saved, gpa_operand dout,
                          gpa_operand dq, hipStream_t stream);

/* Allocation-free forward scan.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  It computes what
 * gpa_gdn_forward computes -- `out` (problem dtype) when q.ptr != NULL and the
 * final state, contiguous [batch,heads,K,V] float32 -- with the forward's
 * intermediates in a static device array of GPA_NOALLOC_SCRATCH_BYTES that
 * each device holds until the process ends, instead of caller buffers (no
 * backward follows).  A problem whose intermediates exceed the array is
 * rejected with GPA_HIP_EINVAL; at K = V = 128 in bf16 that is about 190
 * stream-chunks (e.g. 16 streams of 704 tokens).  It calls no hipMalloc or
 * hipFree.  Every call on a device shares that device's array: calls that
 * overlap in time on one device (two streams, two threads) race. */
#define GPA_NOALLOC_SCRATCH_BYTES (64ull << 20)
int gpa_gdn_scan_noalloc(const gpa_gdn_problem *problem, gpa_operand out, float *final_state,
                         hipStream_t stream);

/* One token of every stream without saved intermediates (inference decode;
 * problem->tokens must be 1, chunk and offset are not used):
 *   final = a S0 + beta u(k) (v - u(k)^T a S0)^T with a = exp(g),
 *   out   = u(q)^T final when q.ptr != NULL,
 * final contiguous [batch,heads,K,V] float32.  With k.ptr == NULL the call
 * only reads: out = u(q)^T S0 (v, g, beta and final unused; q and s0
 * required).  Needs V a multiple of 4, K and V up to 256, s0 and final 16-byte
 * aligned with s0 strides a multiple of 4.  Replaces reference
 * src/gpa/ops.py:29-46 (gdn_update, memory_read), the scan at T = 1 of
 * ops.py:49-85 without the intermediates a backward would need. */
int gpa_gdn_token_step(const gpa_gdn_problem *problem, float *final_state, gpa_operand out, hipStream_t stream);
/* gpa_gdn_token_step of up to GPA_TOKEN_MAX_PACK independent problems
 * (final_states[i], outs[i] belong to problems[i]) in one launch per element
 * type present, every key width (K <= 256) in the same launch: the one-token
 * steps of every relation edge (the _relations loop, attention.py:206-223)
 * or of every level's outer memory (attention.py:333-339) at once.  Results
 * are those of one gpa_gdn_token_step per problem; the problems must not
 * write a state another one reads. */
#define GPA_TOKEN_MAX_PACK 12
int gpa_gdn_token_step_many(const gpa_gdn_problem *problems, float *const *final_states, const gpa_operand *outs,
                            int32_t n, hipStream_t stream);

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

/* ---------------------------------------------------------------- route reader
 * The route reader of one target level j with the default read (reference
 * _bridge, attention.py:225-262, legacy branch :236-240; closed form
 * packed.py:16-35), for every token of every head:
 *   inc   = sum_e w_e m_e                      (w = softmax of the incoming edge logits)
 *   z     = (inc - mean inc) / sqrt(mean (inc - mean inc)^2 + 1e-5)
 *   r0    = softmax(base + gain tanh z)        (rounded to the activation type)
 *   h1    = r0 U,  hd = gelu(h1) D,  r1 = r0 + mlp_gain hd      (= the returned route)
 *   qo    = r1 W_rs + query_scale (q W_qs)
 * with each product's operands and result rounded to the activation type and
 * float32 accumulation, as the reference's typed einsums do.  Rows are the
 * R = batch*tokens token positions; activation tensors are [B,T,H,X] operands
 * whose rows are uniformly strided (sb = tokens*st).
 *
 * Weights are passed pre-padded in the activation type, one [H][N32][K16]
 * matrix per product (N32 = N rounded up to 32, K16 = K rounded up to 16, zero
 * padding), row n holding the contraction over k for output column n:
 *   forward  up_t = U^T [2M][M], down_t = D^T [M][2M], rs_t = W_rs^T [M][M], qs_t = W_qs^T [M][Dk]
 *   backward up = U [M][2M], down = D [2M][M], rs = W_rs [M][M], qs = W_qs [Dk][M]
 * Saved rows (activation type, head-major [H][R][width]): r0 (M), h1 (2M), hd (M). */
#define GPA_ROUTE_MAX_WIDTH 256   /* slots M and key width Dk */
#define GPA_ROUTE_MAX_INCOMING 3
#define GPA_ROUTE_ROWS 32         /* token rows per workgroup; partials have ceil(R/32) rows */

typedef struct gpa_route_problem {
    int32_t batch, tokens, heads, slots, key_dim, incoming, dtype;
    float query_scale;
    gpa_operand base;                             /* float32 [B,T,H,M] base logits */
    gpa_operand msg[GPA_ROUTE_MAX_INCOMING];      /* [B,T,H,M] incoming messages */
    gpa_operand q;                                /* [B,T,H,Dk] */
    const float *edge_weight;                     /* [incoming][H] */
    const float *gain, *mlp_gain;                 /* [H] */
    const void *up_t, *down_t, *rs_t, *qs_t;      /* forward weights (see above) */
    const void *up, *down, *rs, *qs;              /* backward weights */
    gpa_operand qo, route;                        /* outputs [B,T,H,M] */
    void *r0, *h1, *hd;                           /* saved rows */
    /* rsa_update (reference attention.py:251-253): r1 <- round(r1 / clamp(sum|r1|, .25, 4)) per row,
     * in float32, before the query product; the route output is the rescaled row. 0 = off. */
    int32_t rsa;
    /* balanced_bridge (attention.py:256-259): qo = round(mix unit(qr) + (1 - mix) unit(qdir)), with
     * qr = round(r1 W_rs), qdir = round(query_scale round(q W_qs)) and unit(x) = round(x / max(|x|, 1e-6))
     * per row (float32 sums), instead of qo = round(qr + qdir).  0 = off. */
    int32_t balanced;
    const float *mix;                             /* [H]: .1 + .8 sigmoid(bridge_mix_raw) (balanced) */
    void *qr, *qdir;                              /* saved rows [H][R][M] (balanced) */
} gpa_route_problem;

typedef struct gpa_route_grads {
    gpa_operand dqo, droute;                      /* incoming gradients; droute.ptr may be NULL */
    gpa_operand dbase;                            /* float32 out */
    gpa_operand dmsg[GPA_ROUTE_MAX_INCOMING];     /* out */
    gpa_operand dq;                               /* out [B,T,H,Dk] */
    void *dh1, *dhd, *dqs;                        /* out rows [H][R][2M | M | M]: grads of h1, hd and of q W_qs */
    void *hg;                                     /* out rows [H][R][2M]: round(gelu(h1)), read by the weight gradients */
    float *partials;                              /* out [ceil(R/32)][H][2 + incoming]:
                                                     d mlp_gain, d gain, d w_e summed over the block's rows */
    gpa_operand dqr, ddir;                        /* balanced: out rows [H][R][M] addressed as [B,T,H,M]
                                                     (sb = T*M, st = M, sh = R*M): gradients of qr and qdir */
    float *mix_partials;                          /* balanced: out [ceil(R/32)][H], the block's sum of
                                                     dqo . (unit(qr) - unit(qdir)) (d mix after summing) */
} gpa_route_grads;

/* Forward of the route reader.  Replaces the legacy-read body of _bridge
 * (reference attention.py:225-262) and the fused Triton route
 * (triton_route.py:11-151, packed.py:130-136). */
int gpa_route_forward(const gpa_route_problem *problem, hipStream_t stream);
/* The forwards of up to GPA_ROUTE_MAX_PACK problems (the target levels of one
 * call: the same _bridge loop, attention.py:225-262) in one launch where they
 * all take the one-kernel path with the same element type and row access
 * (fewer than 1024 rows each, as in one-token decode); otherwise one
 * gpa_route_forward per problem.  Results are those of gpa_route_forward. */
#define GPA_ROUTE_MAX_PACK 4
int gpa_route_forward_many(const gpa_route_problem *problems, int32_t n, hipStream_t stream);
/* Backward: input and row gradients, plus per-block partial sums of the scalar
 * parameter gradients.  Needs the forward's saved rows and outputs. */
int gpa_route_backward(const gpa_route_problem *problem, const gpa_route_grads *grads, hipStream_t stream);
/* Weight gradients summed over rows, float32 [H][K][N] in the parameters'
 * own layouts: d U [M][2M], d D [2M][M], d W_rs [M][M], d W_qs [Dk][M]
 * (each rounded to the activation type, as the reference's typed products are).
 * Reads the rows dh1, dhd, dqs and hg that gpa_route_backward wrote. */
int gpa_route_weight_grads(const gpa_route_problem *problem, const gpa_route_grads *grads, float *d_up,
                           float *d_down, float *d_rs, float *d_qs, hipStream_t stream);

/* The product relation read of one target level (reference attention.py:
 * 231-236, paper_product_read, with the marginal term of relation_marginal),
 * the part of _bridge before the route softmax; gpa_route_forward then runs
 * on `out` with no incoming messages:
 *   inc  = sum_e (w_e msg_e) n_e        in edge order, n_e = |softmax(source logits)| per row
 *   out  = base + (M gexp) inc  [- gexp log1p(counts)]
 * gexp = e^{clamp(gain, -4, 4)} per head; each product and sum rounded
 * separately, in the reference's order. */
#define GPA_PRODUCT_ROWS 4        /* rows (b, t) of one head per workgroup */
typedef struct gpa_product_problem {
    int32_t batch, tokens, heads, slots, incoming, dtype, marginal;
    gpa_operand base;                             /* float32 [B,T,H,M] */
    gpa_operand msg[GPA_ROUTE_MAX_INCOMING];      /* [B,T,H,M], activation dtype */
    gpa_operand norm[GPA_ROUTE_MAX_INCOMING];     /* float32 [B,T,H] (the last stride is unused) */
    gpa_operand counts;                           /* float32 [B,T,H,M] (marginal only) */
    const float *edge_weight;                     /* [incoming][H] */
    const float *gexp;                            /* [H] */
    float *out;                                   /* float32 [B,T,H,M], contiguous */
} gpa_product_problem;

typedef struct gpa_product_grads {
    const float *dout;                            /* float32 [B,T,H,M], contiguous: gradient of out */
    gpa_operand dmsg[GPA_ROUTE_MAX_INCOMING];     /* out [B,T,H,M], activation dtype */
    float *dnorm[GPA_ROUTE_MAX_INCOMING];         /* out [B,T,H], contiguous */
    float *dcounts;                               /* out [B,T,H,M], contiguous (marginal only) */
    float *partials;                              /* out [ceil(B*T/GPA_PRODUCT_ROWS)][H][2 + incoming]:
                                                     sum dout inc, sum dout log1p(counts), sum d(w_e msg_e) msg_e
                                                     over the workgroup's rows */
} gpa_product_grads;

int gpa_product_read_forward(const gpa_product_problem *problem, hipStream_t stream);
/* d base = dout (not written); d gexp = M * sum(dout inc) - sum(dout log1p(counts)) and
 * d w_e = sum(d(w_e msg_e) msg_e) after summing the partials over their first axis. */
int gpa_product_read_backward(const gpa_product_problem *problem, const gpa_product_grads *grads,
                              hipStream_t stream);

/* ---------------------------------------------------------------- level mix
 * The block-lagged write and residual of one level (reference _block_segment,
 * attention.py:314-329; _residual :190-194), for every token t of block n of
 * every stream, from the block-start snapshots A^_n [Dk][M] and B^_n [M][Dv]:
 *   w   = softmax(u(key) A^_n)                    (rounded to the activation type)
 *   rk  = A^_n w,  rv = w^T B^_n                  (each rounded)
 *   key' = key - eta0 rk,  value' = value - eta1 rv   (rounded)
 * A^_n, B^_n are the scans' chunk-start states (value-major, as gdn_scan
 * saves them) except block 0, which may come from a cached snapshot.  Blocks
 * follow the scan geometry: block n holds tokens n*chunk - offset .. +chunk-1. */
#define GPA_LEVEL_MAX_WIDTH 256     /* key_dim, value_dim and slots */

typedef struct gpa_level_problem {
    int32_t batch, tokens, heads, key_dim, value_dim, slots, chunk, offset, dtype;
    gpa_operand key, value;              /* [B,T,H,Dk], [B,T,H,Dv] */
    const float *a_states, *b_states;    /* [B,H,N][M][Dk] and [B,H,N][Dv][M] float32, contiguous */
    const float *a_first, *b_first;      /* block-0 snapshots [B,H][Dk][M], [B,H][M][Dv], or NULL */
    int64_t a_first_sb, b_first_sb;      /* their batch strides (0: broadcast over the batch) */
    const float *eta;                    /* [H][2]: 1 + .25 tanh(residual_raw[j]) */
    gpa_operand write, key_out, value_out;   /* outputs */
    void *rk, *rv;                       /* saved rounded reconstructions, contiguous [B,T,H,Dk], [B,T,H,Dv] */
    float *stats;                        /* saved softmax row max and sum, contiguous [B,T,H,2] */
    int32_t given_write;                 /* nonzero: `write` is an input (a write that does not read the
                                            snapshots); stats are then neither written nor read */
} gpa_level_problem;

typedef struct gpa_level_grads {
    gpa_operand dwrite, dkey_out, dvalue_out;  /* incoming; dwrite excludes the rk/rv paths (with
                                                  given_write it may be null: zero) */
    gpa_operand dkey;                          /* out: the gradient of key through this step */
    float *da_states, *db_states;              /* out, layouts of a_states / b_states (block 0 included
                                                  unless a_first is given) */
    float *da_first, *db_first;                /* out when a_first / b_first are given: [B,H][Dk][M], [B,H][M][Dv] */
    float *deta;                               /* out [B*H*N][2]: per-block sums of d eta0, d eta1 */
    gpa_operand dwrite_given;                  /* out when problem->given_write: the gradient of the
                                                  given write, dwrite + (drk A^ + drv B^T) rounded;
                                                  dkey is then not written (it equals dkey_out) */
} gpa_level_grads;

/* Forward / backward of the level write and residual (the reference's level
 * glue at attention.py:314-329, autograd through it for the backward).  With
 * given_write the write comes from the slot products (rsa_update's
 * softmax(slot / .25), or softmax slot features: attention.py:186-188) and the
 * kernels form only the reconstructions and the residual step. */
int gpa_level_forward(const gpa_level_problem *problem, hipStream_t stream);
int gpa_level_backward(const gpa_level_problem *problem, const gpa_level_grads *grads, hipStream_t stream);

/* The level write and residual of ONE token of every stream (inference
 * decode; problem->tokens must be 1) from the block snapshots a_first and
 * b_first, which are required (a_states, b_states, rk, rv and stats are not
 * used): write = softmax(u(key) A^) rounded to the activation type,
 * key_out = key - eta0 round(A^ write), value_out = value - eta1 round(write^T B^).
 * With key_out and value_out both null the write alone is formed and B^ is
 * not read (the last level, whose residual nothing reads; shapes of the
 * register kernel only, e.g. Dk = 128 with M up to 256).  given_write is
 * not taken (EUNSUPPORTED).
 * Replaces reference src/gpa/attention.py:314-329 and :190-194 at T = 1. */
int gpa_level_token_forward(const gpa_level_problem *problem, hipStream_t stream);
/* A level's inner one-token step and its one-token level write in one launch
 * (inference decode, reference attention.py:309-329 at T = 1: the A_j update
 * and read, ops.py:29-46, beside _block_segment's write and residual).  The
 * two share no buffers: `step` reads the running state s0 and writes
 * final_state / out, `level` reads the block snapshots.  Results are those of
 * gpa_gdn_token_step(step, final_state, out) and gpa_level_token_forward(level);
 * shapes outside the one-launch kernel (it covers the 512-thread level kernel,
 * e.g. Dk = M = Dv = 128, and key widths 65..256) take those two launches. */
int gpa_token_level_forward(const gpa_gdn_problem *step, float *final_state, gpa_operand out,
                            const gpa_level_problem *level, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Slot counts and base logits of one level (reference attention.py:196-204,
 * with the counts of :318-319, for the default flags):
 *   counts[t] = count0 + sum_{t' <= t} write[t']              (float32)
 *   logits[t] = scale[h] raw[t] + gain[h] log1p(counts[t])
 * The counts are not materialised: the forward writes the logits, the final
 * counts and the counts before every 64-token tile (`prefix`, kept for the
 * backward).  Widths up to 256 slots.
 */
typedef struct gpa_count_problem {
    int32_t batch, tokens, heads, slots, dtype;   /* dtype of raw and write */
    gpa_operand raw, write;                       /* [B,T,H,M] */
    const float *count0;                          /* [B,H,M] at count0[b*count0_sb + h*M + m] */
    int64_t count0_sb;
    const float *gain, *scale;                    /* [H]: softplus(count gain), read scale */
    float *logits;                                /* out [B,T,H,M] float32, contiguous */
    float *final_count;                           /* out [B,H,M] */
    float *prefix;                                /* out/saved [B,H,ceil(T/64),M] */
} gpa_count_problem;

typedef struct gpa_count_grads {
    const float *dlogits;                         /* [B,T,H,M] float32, contiguous */
    const float *dfinal;                          /* [B,H,M] or NULL */
    gpa_operand draw, dwrite;                     /* out [B,T,H,M] (problem dtype) */
    float *dcount0;                               /* out [B,H,M], or NULL */
    float *partials;                              /* out [B*H*ceil(T/64)][2]: d gain, d scale per tile */
    float *tsum;                                  /* scratch [B,H,ceil(T/64),M] */
} gpa_count_grads;

int gpa_count_logits_forward(const gpa_count_problem *problem, hipStream_t stream);
int gpa_count_logits_backward(const gpa_count_problem *problem, const gpa_count_grads *grads,
                              hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Slot products and gate inputs of one level (bf16 activations):
 *   slot = k C^T                 reference attention.py:176-177 (_slot; the
 *                                linear slot feature is the identity)
 *   raw  = unit(k) W_g           attention.py:165 (_gates without control
 *                                input or rsa_update; unit as ops.py:14-17)
 * C = center[level] and W_g = gate_weight[level] rounded to bf16; products
 * accumulate in float32 and round to bf16.  The gate nonlinearities stay with
 * the caller.  Key width a multiple of 16 up to 256, slots a multiple of 32 up
 * to 256, key and dslot rows 16-byte aligned. */
typedef struct gpa_slot_problem {
    int batch, tokens, heads, key_dim, slots, dtype;
    gpa_operand key;                              /* [B,T,H,Dk] */
    const void *center;                           /* [H][M][Dk] bf16 */
    const void *center_t;                         /* [H][Dk][M] bf16 (backward only) */
    const void *gate_w;                           /* [H][Dk][4] bf16 */
    gpa_operand slot, raw;                        /* out [B,T,H,M], [B,T,H,4] (forward) */
} gpa_slot_problem;

typedef struct gpa_slot_grads {
    gpa_operand dslot, draw;                      /* incoming [B,T,H,M], [B,T,H,4] bf16 */
    gpa_operand dkey;                             /* out [B,T,H,Dk]: both terms, added */
    float *dcenter;                               /* out [H][M][Dk], sums rounded to bf16 values */
    float *dgate_w;                               /* out [H][Dk][4], sums rounded to bf16 values */
} gpa_slot_grads;

int gpa_slot_gates_forward(const gpa_slot_problem *problem, hipStream_t stream);
int gpa_slot_gates_backward(const gpa_slot_problem *problem, const gpa_slot_grads *grads, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Element-wise glue of the inference path (no autograd), one launch each.
 *
 * Gate nonlinearities of one level for every token (reference _gates,
 * attention.py:166-174, after the gate-input product):
 *   x = float(raw) + bias;   g_in  = -min(softplus(x0), 10) * decay_scale
 *   b_in  = beta_max sigmoid(x1);   g_out = -min(softplus(x2), 10) * decay_scale
 *   b_out = beta_max sigmoid(x3)
 * decay_scale: 0 for positional_mode "none", the rsa tier, otherwise 1.
 * Outputs: float32 [B,T,H], contiguous. */
typedef struct gpa_gate_problem {
    int32_t batch, tokens, heads, dtype;
    gpa_operand raw;                              /* [B,T,H,4] gate inputs */
    const float *bias;                            /* [H][4] */
    float beta_max, decay_scale;
    float *g_in, *b_in, *g_out, *b_out;           /* out [B,T,H] */
} gpa_gate_problem;
int gpa_gate_act_forward(const gpa_gate_problem *problem, hipStream_t stream);

/* Backward of gpa_gate_act_forward (the autograd of the gate nonlinearities):
 * the four output gradients (float32 [B,T,H], NULL = zero) give draw (the
 * gate inputs' gradient, [B,T,H,4] in dtype) and dbias, partial sums
 * [ceil(B*T*H/256)][H][4] (the caller sums the rows).  heads <= GPA_GATE_MAX_HEADS. */
#define GPA_GATE_MAX_HEADS 256
typedef struct gpa_gate_grads {
    const float *dg_in, *db_in, *dg_out, *db_out;
    gpa_operand draw;
    float *dbias;
} gpa_gate_grads;
int gpa_gate_act_backward(const gpa_gate_problem *problem, const gpa_gate_grads *grads, hipStream_t stream);

/* gpa_slot_gates_forward followed by gpa_gate_act_forward on its gate inputs,
 * in one launch (inference): the slot products and gate inputs of one level
 * (attention.py:176-177, :165) and the gate nonlinearities of _gates
 * (attention.py:161-174).  `gates` gives the bias, beta_max, decay_scale and
 * the four [B,T,H] outputs; its raw operand is not read (the gate inputs are
 * problem->raw, still written).  Results are those of the two calls. */
int gpa_slot_gates_act_forward(const gpa_slot_problem *problem, const gpa_gate_problem *gates,
                               hipStream_t stream);

/* A level's slot products and gates formed inside its one-token inner step
 * (inference decode; bf16 activations, gates from unit(k): no control input,
 * no rsa_update): the step's value is slot = round(k C^T) and its decay and
 * strength are the gate nonlinearities of round(unit(k) W_g), the results of
 * gpa_slot_gates_act_forward (attention.py:161-177), which are also written
 * out (slot, and the four gates for the level's outer step).  The step
 * problem's v, g and beta are not read.  K a multiple of 32 up to 128 (of 64
 * up to 256), M = the step's V a multiple of 4 up to 256. */
typedef struct gpa_token_slot {
    const void *center;          /* [H][M][K] bf16, 16-byte aligned */
    const void *gate_w;          /* [H][K][4] bf16 */
    gpa_gate_problem gates;      /* bias, beta_max, decay_scale, the four [B,1,H] outputs (raw is not read) */
    gpa_operand slot;            /* out [B,1,H,M] bf16 */
} gpa_token_slot;
/* gpa_gdn_token_step (level NULL) or gpa_token_level_forward with the step's
 * value and gates formed in the step as above.  Replaces reference
 * attention.py:309-311 (_slot, _gates) and ops.py:29-46 at T = 1 (with
 * :314-329 when level is given). */
int gpa_token_slot_step(const gpa_gdn_problem *step, const gpa_token_slot *slot, float *final_state,
                        gpa_operand out, const gpa_level_problem *level, hipStream_t stream);

/* One token (T = 1) of one level's slot counts, base logits and local read
 * distribution (attention.py:316-317, _base_logits :196-204, the softmax of
 * :330): n = count0 + write;  logits = scale raw + gain log1p(n);
 * local = softmax(logits) rounded to the activation type. */
#define GPA_TOKEN_LOGITS_MAX_SLOTS 256
typedef struct gpa_token_logits_problem {
    int32_t batch, heads, slots, dtype;
    gpa_operand raw, write;                       /* [B,1,H,M] */
    const float *count0;                          /* [B,H,M] (head slices contiguous) */
    int64_t count0_sb;                            /* its batch stride (0: broadcast) */
    const float *gain, *scale;                    /* [H] */
    float *logits;                                /* out [B,1,H,M] float32, contiguous */
    float *count;                                 /* out [B,H,M], contiguous */
    void *local;                                  /* out [B,1,H,M], contiguous */
} gpa_token_logits_problem;
int gpa_token_logits_forward(const gpa_token_logits_problem *problem, hipStream_t stream);

/* gpa_token_logits_forward of up to GPA_TOKEN_LOGITS_MAX_PACK levels in one
 * launch (every level of one decode step: their logits are read only after
 * the level pass).  Results are those of one call per problem. */
#define GPA_TOKEN_LOGITS_MAX_PACK 8
int gpa_token_logits_many(const gpa_token_logits_problem *problems, int32_t n, hipStream_t stream);

/* Output mix (attention.py:340-341): out = sum_j w[j][h] read_j, in level
 * order, rounded to the activation type. */
typedef struct gpa_mix_problem {
    int32_t batch, tokens, heads, value_dim, levels, dtype;
    gpa_operand read[GPA_DECODE_MAX_LEVELS];      /* [B,T,H,Dv] per level */
    const float *weights;                         /* [L][H] float32 */
    gpa_operand out;                              /* [B,T,H,Dv] */
} gpa_mix_problem;
int gpa_output_mix_forward(const gpa_mix_problem *problem, hipStream_t stream);

/* Backward of the output mix (its autograd, attention.py:340-341):
 * dread_j = round(w[j][h] dout) and dweights [ceil(B*T/32)][levels][heads],
 * per-32-token partial sums of sum dout read_j (the caller sums the tiles).
 * heads <= GPA_MIX_MAX_HEADS; value_dim a multiple of 16 bytes, every row
 * 16-byte aligned; heads*value_dim at most 512 such vectors. */
#define GPA_MIX_MAX_HEADS 256
typedef struct gpa_mix_grads {
    gpa_operand dout;                             /* [B,T,H,Dv] in dtype */
    gpa_operand dread[GPA_DECODE_MAX_LEVELS];     /* out [B,T,H,Dv] in dtype */
    float *dweights;                              /* out, see above */
} gpa_mix_grads;
int gpa_output_mix_backward(const gpa_mix_problem *problem, const gpa_mix_grads *grads, hipStream_t stream);

/* Softmax over rows of float32 logits rounded to dtype, y = round(softmax(x))
 * (the local read distribution softmax(logits).to(dtype), attention.py:330),
 * x and y contiguous [rows][m], 1 <= m <= 1024; and its backward dx = s (dy -
 * sum s dy) with s = softmax(x) recomputed in float32, dy in dtype. */
int gpa_row_softmax_forward(const float *x, void *y, int64_t rows, int32_t m, int32_t dtype, hipStream_t stream);
int gpa_row_softmax_backward(const float *x, const void *dy, float *dx, int64_t rows, int32_t m, int32_t dtype,
                             hipStream_t stream);
/* Device-to-device copies of up to GPA_COPY_MAX buffers in one launch: dst[i]
 * <- src[i], bytes[i] each, every pointer and size a multiple of 16 bytes
 * (GPA_HIP_EINVAL otherwise).  No reference counterpart: it moves a decode
 * token's q, k and v into the buffers a captured decode graph reads. */
#define GPA_COPY_MAX 4
int gpa_copy_many(void *const *dst, const void *const *src, const int64_t *bytes, int32_t n, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Gated moment scan: the per-token recurrence of the additive positional
 * moments (reference src/gpa/ops.py:88-118, `linear_scan`: no gate) and of
 * the counted core's moment and count scans (src/gpa/paper_dense.py:16-58,
 * `moment_scan` and `decayed_counts`).  Per stream, tokens ascending:
 *     S_t = a_t o S_{t-1} + k_t v_t^T,   y_t = S_t^T q_t,   a_t = exp(g_t)
 * where the decay a_t is 1 (GPA_GATE_NONE), one value per token (g [B,T,H]),
 * one per key row (g [B,T,H,K]: row k of S scaled by a_t[k]) or one per value
 * column (g [B,T,H,V]).  No normalisation of q, k or v.  With reverse = 1 the
 * tokens run descending and each step is S += k_t v_t^T; y_t = S^T q_t;
 * S = a_t o S: the adjoint recursion D_t = a_{t+1} o D_{t+1} + q_t dy_t^T of
 * the backward, whose three scans (dq forward on the transposed state, dv
 * reverse, dk reverse on the transposed state) are each one problem.  The
 * state is float32 in registers for the whole sequence, `final` receives it
 * after the last step (for reverse, after the decay of token 0). */
#define GPA_GATE_NONE 0
#define GPA_GATE_TOKEN 1
#define GPA_GATE_KEY 2
#define GPA_GATE_VALUE 3
#define GPA_MOMENT_MAX_KDIM 256
#define GPA_MOMENT_MAX_PACK 4

typedef struct gpa_moment_problem {
    int32_t batch, heads;   /* streams = batch*heads */
    int32_t tokens;         /* T >= 1 */
    int32_t kdim, vdim;     /* 1..GPA_MOMENT_MAX_KDIM rows; vdim >= 1 columns */
    int32_t dtype;          /* GPA_DTYPE_*: q, k, v (and y unless y_f32) */
    int32_t gate;           /* GPA_GATE_* */
    int32_t reverse;        /* 0 ascending, 1 descending (adjoint order) */
    int32_t y_f32;          /* 1: y is float32 */
    int32_t pad_;
    gpa_operand q, k, v;    /* [B,T,H,K], [B,T,H,K], [B,T,H,V] */
    gpa_operand g;          /* float32 log-decay: [B,T,H] (d = 0), [B,T,H,K] or [B,T,H,V]; unused for NONE */
    gpa_operand y;          /* out [B,T,H,V] */
    const float *s0;        /* [B,H,K,V] key-major at s0[b*s0_sb + h*s0_sh + k*V + v]; NULL = zeros */
    int64_t s0_sb, s0_sh;
    float *final;           /* out [B,H,K,V] contiguous float32; NULL = not written */
} gpa_moment_problem;

/* Up to GPA_MOMENT_MAX_PACK independent problems (any widths, gates and
 * directions, one element type) in one launch; the forward is one problem,
 * the backward three.  Results are those of one call per problem. */
int gpa_moment_scan_many(const gpa_moment_problem *problems, int32_t n, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Quadratic Q/K feature map (reference src/gpa/features.py:8-25, applied to q
 * and k by DenseGPA.forward when quadratic_features is set):
 *     u = unit(x) (rounded to dtype),  a = u L_h,  b = u R_h (dtype products),
 *     z = u + gain[h] a b,  out = unit(z) sqrt(sum x^2 + 1e-12)
 * with gain[h] = 2 sigmoid(gain_raw[h]) sqrt(dim) (float32).  x and out are
 * [rows][heads][dim]: row r of head h at x[r*row_stride + h*dim] (out, dout
 * and dx contiguous, row stride heads*dim).  The weights come in two
 * caller-made copies in dtype, zero-padded to DP = ceil(dim/32)*32:
 *     wt [heads][2][DP][DP]:  wt[h][p][n][k] = W_p[h][k][n]  (W_0 = L, W_1 = R)
 *     w  [heads][DP][2*DP]:   w[h][k][p*DP + n] = W_p[h][k][n]
 * The backward writes dx, u ([heads][rows][DP], zero past dim) and d(a)|d(b)
 * ([heads][rows][2*DP]) for the weight gradients dW_p = u^T d(W_p u) (a plain
 * batched product the caller runs), and dgain [ceil(rows/32)][heads]: partial
 * sums of d(gain) per 32-row tile. */
#define GPA_QUAD_MAX_DIM 256

typedef struct gpa_quad_problem {
    int32_t rows, heads, dim, dtype;
    const void *x;
    int64_t row_stride;
    const void *wt, *w;
    const float *gain;      /* [heads] */
    void *out;              /* forward output; unused by the backward */
} gpa_quad_problem;

typedef struct gpa_quad_grads {
    const void *dout;
    void *dx, *u, *dab;
    float *dgain;
} gpa_quad_grads;

int gpa_quad_features_forward(const gpa_quad_problem *problem, hipStream_t stream);
int gpa_quad_features_backward(const gpa_quad_problem *problem, const gpa_quad_grads *grads, hipStream_t stream);

/* dst = src[0] + ... + src[n-1] elementwise over `count` elements of dtype,
 * accumulated in float32 and rounded once; 1 <= n <= GPA_SUM_MAX, every
 * pointer 16-byte aligned and count a whole number of 16-byte vectors (dst may
 * be one of the sources).  No reference counterpart: autograd sums the
 * gradients of an input that several groups of one packed scan call read
 * (reference packed.py:121, a level's write feeds six relation edges) with
 * pairwise adds; the packed call's backward forms that sum in one pass. */
#define GPA_SUM_MAX 8
int gpa_sum_many(void *dst, const void *const *src, int32_t n, int64_t count, int32_t dtype, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* GPA_HIP_H */
