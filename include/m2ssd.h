/*
 * m2ssd.h -- C ABI of libm2ssd.so: the Mamba2 SSD chunked-scan forward and the
 * selective-state-update decode step, as hand-written HIP kernels for MI355X
 * (gfx950).
 *
 * Every entry point takes one argument struct of plain device pointers, sizes
 * and flags, plus a stream (a hipStream_t passed as void*; NULL = the default
 * stream).  Nothing here allocates device memory: outputs and workspace are
 * owned by the caller.  Calls only enqueue work on the stream and never
 * synchronise.  Entry points are re-entrant; errors are reported through the
 * return code and a thread-local message (m2_last_error).
 *
 * Tensor layouts are the reference's (row-major, contiguous):
 *   b = batch, L = seqlen, H = nheads, G = ngroups, P = headdim, N = dstate,
 *   Q = chunk_size, nc = ceil(L / Q).
 * Element types: M2_F32 or M2_BF16 as named per field.  A, D, dt_bias and all
 * state / cumsum / output tensors not marked otherwise are float32.
 */
#ifndef M2SSD_H
#define M2SSD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define M2SSD_ABI_VERSION 5

/* return codes */
#define M2_OK               0
#define M2_ERR_INVALID     -1   /* bad shape, size, pointer or flag */
#define M2_ERR_UNSUPPORTED -2   /* dtype / size this build does not handle */
#define M2_ERR_LAUNCH      -3   /* HIP launch / runtime error */
#define M2_ERR_WORKSPACE   -4   /* workspace missing or too small */

/* element types */
#define M2_F32  0
#define M2_BF16 1

/* ---------------------------------------------------------------------------
 * chunk_cumsum: dt' = clip(softplus?(dt + dt_bias), dt_min, dt_max) (0 past
 * the end of the sequence); dA_cumsum = inclusive cumsum over each chunk of
 * dt' * A.
 * Replaces chunk_cumsum_fwd (reference kernels/chunk_cumsum_fwd.py:288-302,
 * :194-235; naive ops/ssd_naive.py:26-70).
 * ------------------------------------------------------------------------- */
typedef struct {
    const void*  dt;          /* [b, L, H], dt_dtype                     */
    const float* A;           /* [H]                                     */
    const float* dt_bias;     /* [H] or NULL                             */
    float*       dA_cumsum;   /* out [b, H, nc, Q]                       */
    float*       dt_out;      /* out [b, H, nc, Q]                       */
    int64_t batch, seqlen, nheads, chunk_size;
    int32_t dt_dtype;
    int32_t dt_softplus;      /* 0 / 1                                   */
    float   dt_min, dt_max;   /* dt_limit                                */
} m2_chunk_cumsum_args;
int m2_chunk_cumsum(const m2_chunk_cumsum_args* a, void* stream);

/* ---------------------------------------------------------------------------
 * chunk_state: states[b,c,h] = sum_q exp(min(dA[Q-1]-dA[q],0)) dt[q] x[q]^T B[q]
 * (P x N per chunk and head; B shared by the heads of a group).  With seq_idx,
 * positions whose sequence differs from the one at the chunk's last valid
 * position (or where that id is negative) are left out.  Sizes: headdim 32 /
 * 64 / 128, dstate 64 / 128 / 256, chunk_size a multiple of 16 up to 256 (the
 * Python layer maps every other head dim and dstate onto these).
 * Replaces chunk_state_fwd (reference kernels/chunk_state_fwd.py:424-441,
 * :194-304; naive ops/ssd_naive.py:77-128).
 * ------------------------------------------------------------------------- */
typedef struct {
    const void*    x;          /* [b, L, H, P], dtype                    */
    const void*    B;          /* [b, L, G, N], dtype                    */
    const float*   dt;         /* [b, H, nc, Q]                          */
    const float*   dA_cumsum;  /* [b, H, nc, Q]                          */
    const int32_t* seq_idx;    /* [b, L] or NULL                         */
    float*         states;     /* out [b, nc, H, P, N]                   */
    int64_t batch, seqlen, nheads, headdim, ngroups, dstate, chunk_size;
    int32_t dtype;             /* of x and B                             */
} m2_chunk_state_args;
int m2_chunk_state(const m2_chunk_state_args* a, void* stream);

/* ---------------------------------------------------------------------------
 * state_passing: out[:, 0] = initial (or 0); out[:, c+1] = exp(dA[c]) out[:, c]
 * + states[:, c]; final = the value after the last chunk.  With seq_idx the
 * carried state is dropped at chunk c when seq_idx at the end of chunk c
 * differs from seq_idx at the end of chunk c-1 (taken as 0 for c = 0).
 * dA_chunk_cumsum may be a strided view (e.g. dA_cumsum[..., -1]).
 * Replaces state_passing_fwd (reference kernels/state_passing_fwd.py:348-363,
 * :158-341; naive ops/ssd_naive.py:135-182).
 * ------------------------------------------------------------------------- */
typedef struct {
    const float*   states;           /* [b, nc, H, D]                    */
    const float*   dA_chunk_cumsum;  /* [b, H, nc] at the strides below  */
    int64_t        dA_stride_batch, dA_stride_head, dA_stride_chunk;
    const float*   initial_states;   /* [b, H, D] or NULL                */
    const int32_t* seq_idx;          /* [b, seqlen] or NULL              */
    void*          out;              /* out [b, nc, H, D], out_dtype     */
    float*         final_states;     /* out [b, H, D]                    */
    int64_t batch, nchunks, nheads, dim, seqlen, chunk_size;
    int32_t out_dtype;
} m2_state_passing_args;
int m2_state_passing(const m2_state_passing_args* a, void* stream);

/* ---------------------------------------------------------------------------
 * bmm_chunk: out[b,c,g] = a_c @ b_c^T over each chunk (Q x Q, contraction K),
 * then optionally zeroed above the diagonal (causal) and where seq_idx[i] !=
 * seq_idx[j].  k a multiple of 32 (the Python layer zero-pads others),
 * chunk_size a multiple of 16 up to 256.
 * Replaces bmm_chunk_fwd (reference kernels/bmm_chunk_fwd.py:381-400,
 * :293-374; naive ops/ssd_naive.py:189-216).
 * ------------------------------------------------------------------------- */
typedef struct {
    const void*    a;          /* [b, L, G, K], dtype                    */
    const void*    b;          /* [b, L, G, K], dtype                    */
    const int32_t* seq_idx;    /* [b, L] or NULL                         */
    void*          out;        /* out [b, nc, G, Q, Q], out_dtype        */
    int64_t batch, seqlen, ngroups, k, chunk_size;
    int32_t dtype, out_dtype;
    int32_t causal;
} m2_bmm_chunk_args;
int m2_bmm_chunk(const m2_bmm_chunk_args* a, void* stream);

/* ---------------------------------------------------------------------------
 * chunk_scan: out[m] = sum_{k<=m} cb[m,k] exp(dA[m]-dA[k]) dt[k] x[k]
 *                    + exp(dA[m]) C[m] @ states^T + D x[m]; out *= silu(z).
 * states are rounded to x's dtype before use.  out_x (optional) receives the
 * output before the z gate.  With seq_idx, rows whose sequence differs from
 * the one at the previous chunk's last position (0 for chunk 0) get no
 * inter-chunk term; cb is used as given (mask it with bmm_chunk).  Sizes:
 * headdim 32 / 64 / 128, dstate a multiple of 32, chunk_size a multiple of 16
 * up to 256 (the Python layer maps other sizes onto these).
 * Replaces chunk_scan_fwd (reference kernels/chunk_scan_fwd.py:579-600,
 * :482-572; naive ops/ssd_naive.py:223-318).
 * ------------------------------------------------------------------------- */
typedef struct {
    const void*    cb;         /* [b, nc, G, Q, Q], cb_dtype             */
    const void*    x;          /* [b, L, H, P], dtype                    */
    const float*   dt;         /* [b, H, nc, Q]                          */
    const float*   dA_cumsum;  /* [b, H, nc, Q]                          */
    const void*    C;          /* [b, L, G, N], dtype                    */
    const void*    states;     /* [b, nc, H, P, N], states_dtype         */
    const float*   D;          /* [H] or [H, P] or NULL                  */
    const void*    z;          /* [b, L, H, P], dtype, or NULL           */
    const int32_t* seq_idx;    /* [b, L] or NULL                         */
    float*         out;        /* out [b, L, H, P]                       */
    float*         out_x;      /* out [b, L, H, P] or NULL               */
    int64_t batch, seqlen, nheads, headdim, ngroups, dstate, chunk_size;
    int32_t dtype, cb_dtype, states_dtype;
    int32_t D_has_hdim;        /* 1 if D is [H, P]                       */
} m2_chunk_scan_args;
int m2_chunk_scan(const m2_chunk_scan_args* a, void* stream);

/* ---------------------------------------------------------------------------
 * chunk_state_varlen: final state of each packed sequence s (batch 1):
 * the decay-weighted x^T B over its positions in its last chunk, plus
 * exp(dA at its last position) * chunk_states[last chunk] when it started in
 * an earlier chunk.  cu_seqlens is read on the device.
 * Replaces chunk_state_varlen_mosaic (reference kernels/chunk_state_fwd.py:448-597).
 * ------------------------------------------------------------------------- */
typedef struct {
    const void*    B;            /* [L, G, N], dtype                     */
    const void*    x;            /* [L, H, P], dtype                     */
    const float*   dt;           /* [H, nc, Q]                           */
    const float*   dA_cumsum;    /* [H, nc, Q]                           */
    const int32_t* cu_seqlens;   /* [nseq + 1]                           */
    const void*    chunk_states; /* [nc, H, P, N], states_dtype          */
    float*         out;          /* out [nseq, H, P, N]                  */
    int64_t seqlen, nseq, nheads, headdim, ngroups, dstate, nchunks, chunk_size;
    int32_t dtype, states_dtype;
} m2_chunk_state_varlen_args;
int m2_chunk_state_varlen(const m2_chunk_state_varlen_args* a, void* stream);

/* ---------------------------------------------------------------------------
 * ssd_combined: the whole forward (cumsum -> chunk_state -> state_passing ->
 * bmm_chunk -> chunk_scan [-> varlen states]) on one stream, intermediates in
 * the caller's workspace (size from m2_ssd_combined_workspace_size).
 * states_passed is kept in x's dtype; out and the final states are float32.
 * chunk_size is a tiling choice here as in the reference (the outputs are the
 * same function of the inputs for every chunk size): any positive chunk size
 * is accepted; bf16 chunk sizes the fused kernels do not take run as chunks of
 * 128 when that keeps the whole layer on the fused kernels, fp32 chunks of 256
 * and chunk sizes other than 64 / 128 / 256 run as chunks of 128.  Head dim
 * and dstate: the sizes of m2_chunk_state / m2_chunk_scan (the Python layer
 * maps every other size onto these: zero padding, heads of 64, dstate blocks).
 * Replaces mamba_chunk_scan_combined_fwd (reference kernels/ssd_combined.py:46-203).
 * ------------------------------------------------------------------------- */
typedef struct {
    const void*    x;               /* [b, L, H, P], dtype               */
    const void*    dt;              /* [b, L, H], dt_dtype               */
    const float*   A;               /* [H]                               */
    const void*    B;               /* [b, L, G, N], dtype               */
    const void*    C;               /* [b, L, G, N], dtype               */
    const float*   D;               /* [H] / [H, P] / NULL               */
    const void*    z;               /* [b, L, H, P], dtype, or NULL      */
    const float*   dt_bias;         /* [H] or NULL                       */
    const float*   initial_states;  /* [b, H, P, N] or NULL              */
    const int32_t* seq_idx;         /* [b, L] or NULL                    */
    const int32_t* cu_seqlens;      /* [nseq + 1] or NULL (needs b == 1) */
    float*         out;             /* out [b, L, H, P]                  */
    float*         final_states;    /* out [b, H, P, N] or NULL          */
    float*         varlen_states;   /* out [nseq, H, P, N] or NULL       */
    void*          workspace;
    size_t         workspace_bytes;
    int64_t batch, seqlen, nheads, headdim, ngroups, dstate, chunk_size, nseq;
    int32_t dtype, dt_dtype;
    int32_t D_has_hdim, dt_softplus;
    float   dt_min, dt_max;
    void**         stage_events;    /* optional profiling hook: NULL, or 7
                                       hipEvent_t recorded before stage 1,
                                       after each of the 5 stages and after
                                       the varlen states (when requested); a
                                       NULL entry is not recorded.  With bf16
                                       and the fused scan the varlen states
                                       run after state_passing, so event 6
                                       is recorded before events 4 and 5    */
} m2_ssd_combined_args;
size_t m2_ssd_combined_workspace_size(const m2_ssd_combined_args* a);
int m2_ssd_combined(const m2_ssd_combined_args* a, void* stream);

/* ---------------------------------------------------------------------------
 * m2_ssd_combined without a workspace: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc): the same kernels and
 * results as m2_ssd_combined, with the workspace taken from a static device
 * array of M2_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends);
 * a->workspace / a->workspace_bytes are not read.  Calls no allocating
 * routine.  Problems whose m2_ssd_combined_workspace_size exceeds the array
 * return M2_ERR_WORKSPACE.  Calls that overlap in time on one GPU race on its
 * array; the array keeps the last call's contents.
 * ------------------------------------------------------------------------- */
#define M2_NOALLOC_SCRATCH_BYTES (128u << 20)
int m2_ssd_combined_noalloc(const m2_ssd_combined_args* a, void* stream);
/* Looks up the static array on the current device (what the first
 * m2_ssd_combined_noalloc call there does otherwise).  That lookup may load
 * code onto the device, which a capturing stream must not see: the first
 * m2_ssd_combined_noalloc call on a device refuses a stream under graph
 * capture (M2_ERR_INVALID), so a caller that captures calls this once per
 * device beforehand.  No counterpart in the reference; for the same callers. */
int m2_ssd_combined_noalloc_prepare(void);

/* ---------------------------------------------------------------------------
 * selective_state_update (one decode token):
 * dt' = softplus?(dt + dt_bias); new = state * exp(dt' A) + dt' x B^T;
 * out = new @ C + D x; out *= silu(z).
 * new goes to new_state, or back into state when new_state is NULL (or
 * equal to state): the in-place update of a decode loop that owns its state.
 * Any headdim and dstate (16-byte aligned rows are the fast path: dstate a
 * multiple of 4 up to 256).
 * Replaces selective_state_update (reference ops/selective_state_update.py:22-123).
 * ------------------------------------------------------------------------- */
typedef struct {
    float*       state;        /* [b, H, P, N] (read; written when in place) */
    const void*  x;            /* [b, H, P], dtype                       */
    const void*  dt;           /* [b, H] or [b, H, P], dt_dtype          */
    const float* A;            /* [H] or [H, P, N]                       */
    const void*  B;            /* [b, G, N], dtype                       */
    const void*  C;            /* [b, G, N], dtype                       */
    const float* D;            /* [H] / [H, P] / NULL                    */
    const void*  z;            /* [b, H, P], dtype, or NULL              */
    const float* dt_bias;      /* [H] / [H, P] / NULL                    */
    float*       out;          /* out [b, H, P]                          */
    int64_t batch, nheads, headdim, ngroups, dstate;
    int32_t dtype, dt_dtype;
    int32_t dt_has_hdim, A_full, D_has_hdim, dt_bias_has_hdim;
    int32_t dt_softplus;
    float*       new_state;    /* [b, H, P, N] result, or NULL: into state */
} m2_ssu_args;
int m2_selective_state_update(const m2_ssu_args* a, void* stream);

/* ---------------------------------------------------------------------------
 * Output of a causal_conv1d call: channels [c_begin, next range's c_begin) of
 * the result go to `ptr`, element (b, c, t) at
 *   b * stride_batch + (c - c_begin) * stride_dim + t * stride_time
 * (strides in elements of the result dtype).  One range covers every channel;
 * three ranges write x, B and C of an SSD layer straight into their own
 * tensors.
 * ------------------------------------------------------------------------- */
typedef struct {
    void*   ptr;
    int64_t c_begin;
    int64_t stride_batch, stride_dim, stride_time;
} m2_conv_out;

/* ---------------------------------------------------------------------------
 * causal_conv1d: depthwise causal convolution over time, per channel c:
 *   xm[s] = x[s], zeroed when seq_idx is given and seq_idx[s + j] !=
 *           seq_idx[s + j - 1] for some 1 <= j < width with s + j < L
 *   y[t]  = sum_{i < width} weight[c, i] xm[t - width + 1 + i]  (0 before t = 0)
 *   out   = silu?(y + bias[c])
 * The result dtype (out_dtype) is bf16 when x, weight and bias (if given) are
 * all bf16, else f32; a bf16 conv result is rounded before the bias add.
 * x is addressed through (batch, channel, time) element strides: a contiguous
 * [b, d, L] array and a [b, L, d] channels-last buffer both work (unit channel
 * stride and unit time stride are the fast layouts).
 * Replaces causal_conv1d (reference ops/causal_conv1d.py:18-85, boundary mask
 * :142-193).
 * ------------------------------------------------------------------------- */
typedef struct {
    const void*    x;              /* [b, d, L] at the strides below, x_dtype */
    int64_t        x_stride_batch, x_stride_dim, x_stride_time;
    const void*    weight;         /* [d, width] contiguous, w_dtype          */
    const void*    bias;           /* [d], bias_dtype, or NULL               */
    const int32_t* seq_idx;        /* [b, L] contiguous, or NULL             */
    m2_conv_out    out[3];         /* nout ranges, out[0].c_begin = 0        */
    int64_t batch, dim, seqlen, width;   /* width 1 .. 8                     */
    int32_t nout;
    int32_t x_dtype, w_dtype, bias_dtype, out_dtype;
    int32_t silu;                  /* 0 / 1 (activation="silu")              */
} m2_causal_conv1d_args;
int m2_causal_conv1d(const m2_causal_conv1d_args* a, void* stream);

/* ---------------------------------------------------------------------------
 * causal_conv1d_update (one decode token):
 *   new_state = concat(conv_state[:, :, 1:], x[:, :, None])
 *   out = silu?(sum_i new_state[:, :, i] weight[:, i] + bias)
 * new_state_dtype is bf16 when conv_state and x are bf16, else f32; new_state
 * may be conv_state (in-place update, same dtype).  The products are bf16
 * (each rounded, their sum rounded once) when new_state and weight are bf16;
 * out_dtype is bf16 when those and the bias are bf16, else f32.  The outputs'
 * stride_dim must be 1 (stride_time is ignored).
 * Replaces causal_conv1d_update (reference ops/causal_conv1d.py:88-139).
 * ------------------------------------------------------------------------- */
typedef struct {
    const void* x;                 /* [b, d] at x_stride_batch, x_dtype      */
    int64_t     x_stride_batch;
    const void* conv_state;        /* [b, d, width] contiguous, state_dtype  */
    void*       new_state;         /* [b, d, width] contiguous               */
    const void* weight;            /* [d, width] contiguous, w_dtype         */
    const void* bias;              /* [d], bias_dtype, or NULL               */
    m2_conv_out out[3];            /* nout ranges, out[0].c_begin = 0        */
    int64_t batch, dim, width;     /* width 1 .. 8                           */
    int32_t nout;
    int32_t x_dtype, state_dtype, new_state_dtype, w_dtype, bias_dtype, out_dtype;
    int32_t silu;
} m2_causal_conv1d_update_args;
int m2_causal_conv1d_update(const m2_causal_conv1d_update_args* a, void* stream);

/* ---------------------------------------------------------------------------
 * rms_norm_gated over groups of group_size consecutive elements of each row:
 *   x' = x * silu(z)                 (z given and !norm_before_gate)
 *   out = x' / sqrt(mean(x'^2) + eps) * weight
 *   out = out * silu(z)              (z given and norm_before_gate)
 * Every intermediate is bf16 exactly when all its operands are (x, z, weight
 * as they enter it); out_dtype is that result dtype, or bf16 (the result
 * rounded at the store, for a bf16 consumer such as a projection).  Rows are addressed
 * through row strides (elements; the last dimension is contiguous), e.g. z as
 * a slice of the in-projection output.
 * Replaces rms_norm_gated (reference ops/rms_norm.py:15-92).
 * ------------------------------------------------------------------------- */
typedef struct {
    const void* x;                 /* [rows, hidden] at x_row_stride, x_dtype   */
    const void* z;                 /* [rows, hidden] at z_row_stride, or NULL   */
    const void* weight;            /* [hidden], w_dtype                         */
    void*       out;               /* [rows, hidden] at out_row_stride          */
    int64_t x_row_stride, z_row_stride, out_row_stride;
    int64_t rows, hidden, group_size;   /* group_size divides hidden          */
    float   eps;
    int32_t x_dtype, z_dtype, w_dtype, out_dtype;
    int32_t norm_before_gate;      /* 0 / 1                                     */
    float*  residual;              /* [rows, hidden] f32 or NULL: with z == NULL,
                                      residual += x (stored back) and the sum is
                                      normalised (a pre-norm block's residual add) */
    int64_t residual_row_stride;
} m2_rms_norm_gated_args;
int m2_rms_norm_gated(const m2_rms_norm_gated_args* a, void* stream);

/* ---------------------------------------------------------------------------
 * skinny_gemm: y[M, N] = x[M, K] w[N, K]^T (+ bias[N]) for M <= 64, bf16 x and w
 * (K-contiguous rows: the [out, in] layout of a linear layer), float32
 * accumulation, y in bf16 or f32.  No counterpart operator in the reference
 * (whose projections are XLA GEMMs, modules/mamba2.py:464-469, :538-541,
 * models/mamba2_lm.py:699, :734): the decode step's in-/out-projections and LM
 * head, which are bound by reading the weights once per token.
 * K and the x / w row strides must be multiples of 8 (16-byte rows).
 * ------------------------------------------------------------------------- */
typedef struct {
    const void* x;                 /* [M, K] at ldx, bf16                       */
    const void* w;                 /* [N, K] at ldw, bf16                       */
    const void* bias;              /* [N], bias_dtype, or NULL                  */
    void*       y;                 /* out [M, N] at ldy, y_dtype                */
    int64_t M, N, K, ldx, ldw, ldy;
    int32_t x_dtype, w_dtype, bias_dtype, y_dtype;
} m2_skinny_gemm_args;
int m2_skinny_gemm(const m2_skinny_gemm_args* a, void* stream);

/* ---------------------------------------------------------------------------
 * skinny_gemm_norm: y = rms_norm_gated(x, norm_weight, z)[M, K] w[N, K]^T
 * (+ bias) for M <= 16 and M * K <= 32768: m2_skinny_gemm whose input rows are
 * normalised first, with m2_rms_norm_gated's arithmetic (groups of group_size
 * <= 8 per row, the optional SiLU gate z before / after the norm, the
 * reference's rounding points) and stored as bf16 -- done by every
 * workgroup in its own LDS, so the norm takes no launch and no round trip.
 * With residual != NULL the result (rounded to y_dtype) is added into the f32
 * residual rows; y may then be NULL.  No counterpart operator in the
 * reference: it fuses the pre-norm / gated norm of a decode step into the
 * projection that follows (reference models/mamba2_lm.py:205-211 and
 * modules/mamba2.py:536-541), for decode loops that are bound by launch
 * latency.  Group, stride and base alignment: 4 elements.
 * ------------------------------------------------------------------------- */
typedef struct {
    const void* x;                 /* [M, K] at x_row_stride, x_dtype            */
    const void* z;                 /* [M, K] at z_row_stride, z_dtype, or NULL   */
    const void* norm_weight;       /* [K], norm_weight_dtype                     */
    int64_t x_row_stride, z_row_stride, group_size;
    float   eps;
    int32_t x_dtype, z_dtype, norm_weight_dtype, norm_before_gate;
    const void* w;                 /* [N, K] at ldw, bf16                        */
    const void* bias;              /* [N], bias_dtype, or NULL                   */
    void*       y;                 /* out [M, N] at ldy, y_dtype, or NULL        */
    float*      residual;          /* [M, N] f32 at residual_row_stride, or NULL:
                                      residual += y                              */
    int64_t M, N, K, ldw, ldy, residual_row_stride;
    int32_t w_dtype, bias_dtype, y_dtype;
    /* with_conv: the decode conv update (m2_causal_conv1d_update) of output
       columns [conv_begin, conv_begin + conv.dim), run on each column once it
       is computed (rounded to y_dtype); conv.x is not read, conv.batch == M,
       conv.width 4, f32 conv_state updated in place (new_state == conv_state) */
    int32_t with_conv;
    int64_t conv_begin;
    m2_causal_conv1d_update_args conv;
} m2_skinny_gemm_norm_args;
int m2_skinny_gemm_norm(const m2_skinny_gemm_norm_args* a, void* stream);

/* ---------------------------------------------------------------------------
 * Testing hook, no counterpart in the reference: forces one of the kernel
 * choices the library otherwise makes from the shape, process-wide, so that a
 * test can run every path on one shape (production code never calls it; no
 * environment variable is read).  value 0 restores the automatic choice; a
 * forced choice the shape cannot take is ignored.  Returns the previous value,
 * or M2_ERR_INVALID for an unknown knob or value.
 * ------------------------------------------------------------------------- */
#define M2_KNOB_STATES_SPLIT  0   /* bf16 fused state pass: 1 a head in 64-column
                                     halves, 2 head pairs x 64 columns, 3 head
                                     pairs x 128 columns                       */
#define M2_KNOB_F32_STATES    1   /* fp32 layer: 1 the fused state pass, 2 the
                                     staged chunk_state + state_passing        */
#define M2_KNOB_ONESHOT_HEADS 2   /* one-shot state kernel: 1 one head per
                                     workgroup                                 */
#define M2_KNOB_F32_SCAN      3   /* fp32 chunk_scan (chunk 128, head dim 64):
                                     1 one workgroup per (chunk, head); v >= 2
                                     one per (chunk, group, slice of v - 1 of
                                     the group's heads)                        */
int m2_set_dispatch_override(int knob, int value);

/* thread-local message for the last non-zero return code of this thread */
const char* m2_last_error(void);
/* M2SSD_ABI_VERSION of the loaded library */
int m2_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* M2SSD_H */
