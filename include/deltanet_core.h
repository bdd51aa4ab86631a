/* deltanet_core.h — C ABI of the MI355X (gfx950) delta-rule core.
 *
 * Drop-in boundary for burn-deltanet's delta-rule core (Rust crate
 * `burn-deltanet` v0.14.0). Three entry points replace the reference's three
 * interfaces on the hot path:
 *
 *   dn_chunk_fwd  ← DeltaChunkBackendExt::delta_chunk_recalculated
 *                   (src/delta/chunk_recalculated/chunk_recalculated.rs:86-151;
 *                    reached through DeltaInput::run, src/delta/path.rs:215-231)
 *   dn_step       ← delta_step (src/delta/recurrent.rs:41-99)
 *   dn_chunk_bwd  ← combined_backward
 *                   (src/delta/chunk_recalculated/combined_backward.rs:72-189,
 *                    called from the autodiff node, backward.rs:82-170)
 *
 * Around them: dn_recurrent (DeltaInput::delta_recurrent), dn_frontend and
 * dn_out_norm (the families' projection front-end and output norm) and
 * dn_unit_lower_inverse (the public unit_lower_inverse, src/delta/tri.rs).
 *
 * Conventions (src/delta/path.rs:120-141). All tensors are dense row-major
 * device buffers in the reference's axis order:
 *   q, k      [batch, sequence, nheads, head_k_dim]      dtype qkv_dtype
 *   v         [batch, sequence, nheads, head_v_dim]      dtype qkv_dtype
 *   erase     [batch, sequence, nheads, erase_width]     float32, width 1 | head_k_dim
 *   write     [batch, sequence, nheads, write_width]     float32, width 1 | head_v_dim
 *   g         [batch, sequence, nheads, decay_width]     float32, width 1 | head_k_dim,
 *             log forget gate g = log α ≤ 0; read only when has_gate != 0
 *   state     [batch, nheads, head_k_dim, head_v_dim]    float32
 *   y         [batch, sequence, nheads, head_v_dim]      dtype y_dtype
 * For dn_step the `sequence` axis is absent ([batch, nheads, ·]).
 * q and k arrive L2-normalised and unscaled; `scale` is applied to q inside
 * (NaN selects 1/sqrt(head_k_dim), path.rs:161-165). The core applies exp(g)
 * and nothing else to the gates.
 *
 * The reference is functional; here outputs are written to caller buffers.
 * state_out may alias state_in (an in-place update of the state). No other
 * output may alias an input.
 *
 * Every call is asynchronous on `stream` (NULL = the default stream) unless
 * check_finite is set, which synchronises to read the NaN/Inf guard back.
 * Return value: DN_OK or a negative dn_status; dn_last_error() gives the text
 * of the reference's assertion that the status mirrors.
 */
#ifndef DELTANET_CORE_H
#define DELTANET_CORE_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  DN_F32 = 0,
  DN_BF16 = 1,
} dn_dtype;

/* Which kernels run dn_chunk_fwd / dn_chunk_bwd. AUTO picks the MFMA path
 * (DN_ALGO_MFMA) whenever the shape, dtypes and pointers allow it (bf16
 * q/k/v, head_k_dim 64 or 128 with head_v_dim a multiple of 64; with
 * per-head or no gates also head_k_dim 256 with head_v_dim a multiple of
 * 128, forward and backward): q and k
 * (and, for the backward, d_y) at 16-byte boundaries, v at a 4-byte one, and
 * nheads·max(head_k_dim, head_v_dim) below 2^23 (the kernels address a
 * chunk's token rows with 32-bit byte offsets). Otherwise AUTO runs the
 * generic kernels and an explicit MFMA request is refused. */
typedef enum {
  DN_ALGO_AUTO = 0,
  DN_ALGO_GENERIC = 1, /* fp32 arithmetic, any shape */
  DN_ALGO_MFMA = 2,    /* bf16 MFMA tiles; DN_ERR_UNSUPPORTED if the shape does not fit.
                          The forward runs two kernels (intra-chunk tiles through the
                          workspace, then the scan). */
  DN_ALGO_MFMA_FUSED = 3, /* the MFMA forward as one kernel that builds each chunk's WY
                             tiles in LDS beside the scan: q/k/v read once, no tile
                             traffic, a 1 KB workspace instead of the two-kernel path's
                             tiles (203 MB at BASELINE config 2), about 20% slower there.
                             Per-head gates, head_k_dim 128, head_v_dim a multiple of 128,
                             bf16 q/k/v; DN_ERR_UNSUPPORTED otherwise. Never chosen by AUTO;
                             the backward treats it as DN_ALGO_MFMA. */
} dn_algo;

typedef enum {
  DN_OK = 0,
  DN_ERR_SEQUENCE = -1,    /* "sequence length must be at least 1" (path.rs:179) */
  DN_ERR_SHAPE = -2,       /* a dimension < 1, or shapes that disagree (path.rs:180-185,
                              recurrent.rs:51-54) */
  DN_ERR_GATE_WIDTH = -3,  /* "{gate}: last axis must be 1 or {full}" (path.rs:187-197) */
  DN_ERR_CHUNK_LEN = -4,   /* "chunk_len must be at least 1" (path.rs:219); also chunk_len²
                              or chunk_len·max(head_k_dim, head_v_dim) at or above 2^31 */
  DN_ERR_NONFINITE = -5,   /* NaN/Inf guard on inputs or outputs (sanity, path.rs:198-207) */
  DN_ERR_NULL = -6,        /* a required pointer is NULL */
  DN_ERR_DTYPE = -7,       /* unknown dtype tag */
  DN_ERR_WORKSPACE = -8,   /* caller workspace smaller than dn_*_workspace_bytes() */
  DN_ERR_UNSUPPORTED = -9, /* DN_ALGO_MFMA requested for a shape it does not cover */
  DN_ERR_HIP = -10,        /* a HIP runtime call failed */
} dn_status;

/* DeltaChunkBackendExt::delta_chunk_recalculated (chunk_recalculated.rs:115-151). */
typedef struct {
  int64_t batch, sequence, nheads, head_k_dim, head_v_dim;
  int64_t erase_width, write_width, decay_width; /* decay_width ignored when !has_gate */
  int32_t has_gate;
  int32_t chunk_len;     /* tokens per chunk, >= 1; the reference default is 64 */
  double scale;          /* NaN => 1/sqrt(head_k_dim) */
  int32_t qkv_dtype;     /* dn_dtype of q, k, v */
  int32_t y_dtype;       /* dn_dtype of y */
  int32_t algo;          /* dn_algo */
  int32_t check_finite;  /* nonzero: NaN/Inf guard on inputs and outputs (synchronises) */
  const void *q, *k, *v;
  const float *erase, *write, *g;
  const float *state_in;
  void *y;
  float *state_out;
  void *workspace;         /* NULL => library-managed workspace (see below) */
  size_t workspace_bytes;
} dn_chunk_fwd_args;

/* combined_backward (combined_backward.rs:72-189). Same leaves as the forward,
 * plus the two incoming cotangents; writes the seven gradients. d_erase,
 * d_write and d_g are reduced to their gate's own width (forward.rs:106-112);
 * d_g is the gradient with respect to g = log α.
 * On the MFMA path the call forks its reverse scan onto a second stream that
 * the library keeps per (device, calling stream), and joins it back into the
 * calling stream before its last kernel: everything the call does is ordered
 * on `stream`. Callers on different streams get different second streams;
 * under HIP graph capture of `stream` the second stream joins the capture. */
typedef struct {
  int64_t batch, sequence, nheads, head_k_dim, head_v_dim;
  int64_t erase_width, write_width, decay_width;
  int32_t has_gate;
  int32_t chunk_len;
  double scale;
  int32_t qkv_dtype;     /* dtype of q, k, v */
  int32_t grad_dtype;    /* dtype of d_y and of d_q, d_k, d_v */
  int32_t algo;
  int32_t check_finite;
  const void *d_y;               /* [batch, sequence, nheads, head_v_dim] */
  const float *d_state_final;    /* [batch, nheads, head_k_dim, head_v_dim]; NULL = zeros */
  const void *q, *k, *v;
  const float *erase, *write, *g;
  const float *state_in;
  void *d_q, *d_k, *d_v;
  float *d_erase, *d_write, *d_g; /* d_g may be NULL when !has_gate */
  float *d_state;
  void *workspace;
  size_t workspace_bytes;
} dn_chunk_bwd_args;

/* delta_step (recurrent.rs:41-99): one tick for all heads. */
typedef struct {
  int64_t batch, nheads, head_k_dim, head_v_dim;
  int64_t erase_width, write_width, decay_width;
  int32_t has_gate;
  double scale;          /* NaN => 1/sqrt(head_k_dim) */
  int32_t qkv_dtype;
  int32_t y_dtype;
  int32_t check_finite;
  const void *q, *k, *v;        /* [batch, nheads, head_k_dim | head_v_dim] */
  const float *erase, *write, *g;
  const float *state_in;        /* [batch, nheads, head_k_dim, head_v_dim] */
  void *y;                      /* [batch, nheads, head_v_dim] */
  float *state_out;             /* may alias state_in */
} dn_step_args;

/* delta_step over a whole sequence (recurrent.rs:107-142): the same gates and
 * layouts as dn_chunk_fwd, evaluated token by token like the reference's
 * DeltaPath::Recurrent. */
typedef struct {
  int64_t batch, sequence, nheads, head_k_dim, head_v_dim;
  int64_t erase_width, write_width, decay_width;
  int32_t has_gate;
  double scale;          /* NaN => 1/sqrt(head_k_dim) */
  int32_t qkv_dtype;
  int32_t y_dtype;
  int32_t check_finite;
  const void *q, *k, *v;        /* [batch, sequence, nheads, head_k_dim | head_v_dim] */
  const float *erase, *write, *g; /* [batch, sequence, nheads, width] */
  const float *state_in;        /* [batch, nheads, head_k_dim, head_v_dim] */
  void *y;                      /* [batch, sequence, nheads, head_v_dim] */
  float *state_out;             /* may alias state_in */
} dn_recurrent_args;

/* Replaces DeltaChunkBackendExt::delta_chunk_recalculated
 * (src/delta/chunk_recalculated/chunk_recalculated.rs:110-151). */
int dn_chunk_fwd(const dn_chunk_fwd_args *args, hipStream_t stream);

/* Replaces combined_backward
 * (src/delta/chunk_recalculated/combined_backward.rs:72-84). */
int dn_chunk_bwd(const dn_chunk_bwd_args *args, hipStream_t stream);

/* Replaces delta_step (src/delta/recurrent.rs:41-50). */
int dn_step(const dn_step_args *args, hipStream_t stream);

/* Replaces DeltaInput::delta_recurrent (src/delta/recurrent.rs:107-142), the
 * DeltaPath::Recurrent arm of DeltaInput::run (path.rs:215-231): delta_step
 * unrolled over the sequence, with the state kept on chip from the first
 * token to the last (one read and one write of it per call instead of one
 * of each per token). DeltaProduct's decode folds its u Householder
 * micro-steps into a u-token sequence and runs it this way
 * (delta_product.rs:270-305). head_k_dim up to 512; larger returns
 * DN_ERR_UNSUPPORTED (delta_step per token covers it). */
#define DN_RECURRENT_MAX_K 512
int dn_recurrent(const dn_recurrent_args *args, hipStream_t stream);

/* The projection front-end: everything QkvProjection::forward does after its
 * in_proj GEMM (src/common/qkv.rs:373-449), and QkvProjection::step's
 * single-token form (:454-516) as sequence = 1. From the projection output
 * [q | k (u copies) | v (u copies) | beta or (erase | write)] (qkv.rs:237-262)
 * it produces the delta rule's inputs in one pass: the causal depthwise short
 * convolution with its rolling window and fused activation (ShortConv,
 * src/common/conv.rs:85-158), the q/k activation, the q/k L2 norm
 * (norm.rs:36-97), v's SiLU, the head split with the n_householder micro-steps
 * folded into the sequence, and the squashed write gates (squash_write,
 * qkv.rs:332-369). The reference runs these as separate passes over the
 * projection. n_value_heads = nheads only (grouped values replicate heads in
 * burn_stack code the reference does not vendor), and QkNorm::Sum is not
 * offered (its epsilon lives there too): both return DN_ERR_UNSUPPORTED. */
typedef enum {
  DN_ACT_IDENTITY = 0,
  DN_ACT_SILU = 1,
  DN_ACT_RELU = 2,          /* q/k activation only */
  DN_ACT_ELU_PLUS_ONE = 3   /* q/k activation only */
} dn_activation;

typedef enum { DN_QKNORM_NONE = 0, DN_QKNORM_L2 = 1, DN_QKNORM_SUM = 2 } dn_qk_norm;

typedef enum { DN_WRITE_FIXED = 0, DN_WRITE_SCALAR = 1, DN_WRITE_CHANNEL = 2 } dn_write_gate;

typedef struct {
  int64_t batch, sequence;      /* tokens per call; 1 for QkvProjection::step */
  int64_t nheads, head_k_dim, head_v_dim;  /* head dims up to DN_FRONTEND_MAX_HEAD_DIM */
  int64_t n_householder;        /* u >= 1 micro-steps per token (DeltaProduct) */
  int64_t conv_kernel;          /* 0: no short convolution; else 1..DN_FRONTEND_MAX_KERNEL */
  int64_t proj_stride;          /* elements from one token's projection row to the next */
  int32_t conv_activation;      /* DN_ACT_SILU or DN_ACT_IDENTITY */
  int32_t qk_activation;        /* dn_activation */
  int32_t qk_norm;              /* DN_QKNORM_L2 or DN_QKNORM_NONE */
  int32_t write_gate;           /* dn_write_gate */
  int32_t allow_neg_eigval;     /* doubles the erase gate (and the scalar beta) */
  int32_t in_dtype;             /* projected and the windows: DN_F32 or DN_BF16 */
  int32_t out_dtype;            /* q, k, v: DN_F32 or DN_BF16 */
  const void *projected;        /* [batch, sequence, proj_stride] */
  const float *conv_weight;     /* [conv_dim, conv_kernel] (Conv1d's [conv_dim, 1, kernel]) */
  const float *conv_bias;       /* [conv_dim] or NULL */
  const void *window_in;        /* [batch, conv_dim, conv_kernel], newest column last */
  void *window_out;             /* same shape; may alias window_in */
  void *q;                      /* [batch, sequence, nheads, head_k_dim] */
  void *k;                      /* [batch, sequence * u, nheads, head_k_dim] */
  void *v;                      /* [batch, sequence * u, nheads, head_v_dim] */
  float *erase;                 /* [batch, sequence * u, nheads, 1 | head_k_dim] */
  float *write;                 /* [batch, sequence * u, nheads, 1 | head_v_dim]; may equal erase
                                   for DN_WRITE_FIXED / DN_WRITE_SCALAR, where they are one tensor */
} dn_frontend_args;

#define DN_FRONTEND_MAX_HEAD_DIM 256
#define DN_FRONTEND_MAX_KERNEL 8

/* Replaces QkvProjection::forward / ::step after in_proj
 * (src/common/qkv.rs:373-449, 454-516). conv_dim = nheads*head_k_dim +
 * u*nheads*(head_k_dim + head_v_dim) (qkv.rs:180-182); the write-gate columns
 * follow at conv_dim (qkv.rs:267-300). */
int dn_frontend(const dn_frontend_args *args, hipStream_t stream);

/* The output norm after the delta rule: OutNorm::forward
 * (src/common/norm.rs:106-144), per head over head_v_dim. Gated:
 * out = x / sqrt(mean(x^2) + eps) * weight * silu(gate); plain (gate NULL):
 * the same without the gate factor. Both RmsNorm forms live in burn_stack,
 * which the reference does not vendor, so eps is the caller's (burn's RmsNorm
 * default is 1e-5). The gate is read in place from the projection: row t's
 * gate for head h starts at gate + t*gate_stride + h*head_v_dim. */
typedef struct {
  int64_t tokens;               /* batch * sequence (or batch for a decode step) */
  int64_t nheads, head_v_dim;
  int64_t gate_stride;          /* elements between consecutive tokens' gates */
  double eps;
  int32_t x_dtype, gate_dtype, out_dtype;   /* DN_F32 or DN_BF16 */
  const void *x;                /* [tokens, nheads, head_v_dim] */
  const void *gate;             /* NULL for OutNorm::Plain */
  const float *weight;          /* gamma [head_v_dim] */
  void *out;                    /* [tokens, nheads, head_v_dim]; may alias x */
} dn_out_norm_args;

#define DN_OUT_NORM_MAX_HEAD_DIM 1024

/* Replaces OutNorm::forward (src/common/norm.rs:127-134) as called after the
 * delta rule by every family (deltanet.rs:171, 219; gated_deltanet_1.rs:183, 234;
 * gated_deltanet_2.rs:282, 367; delta_product.rs:230, 306). */
int dn_out_norm(const dn_out_norm_args *args, hipStream_t stream);

/* The chunk forward followed by the output norm, as every family runs them
 * over a sequence: DeltaChunkBackendExt::delta_chunk_recalculated
 * (chunk_recalculated.rs:115-151), then OutNorm::forward
 * (src/common/norm.rs:106-144) on its y (gated_deltanet_1.rs:183-186 and the
 * others listed at dn_out_norm). `fwd` as for dn_chunk_fwd, except that
 * fwd.y receives OutNorm's output (dtype fwd.y_dtype) in place of the delta
 * rule's y; the gate, weight and eps as for dn_out_norm, the gate rows
 * [batch, sequence] gate_stride elements apart (a column view of the
 * projection), head h's gates at h*head_v_dim. in_scan = 0 runs the
 * chunk forward and then the norm as a pass of its own over y (in place);
 * in_scan = 1 applies the norm in the MFMA scan's output write, so y makes no
 * round trip through HBM, where the MFMA path runs (AUTO or DN_ALGO_MFMA)
 * and the gate, if any, has y's dtype. The separate pass is the faster of
 * the two at every shape measured on MI355X (0.53 against
 * 0.60 ms): the scan is latency-bound, and the norm's work inside its chunk
 * loop lengthens it more than the pass costs. In the scan, a head's columns
 * may span several workgroups, which then exchange per-token sums of squares
 * during the kernel; that launch is cooperative (the grid must be resident
 * at once), and where the device cannot hold it the call falls back to the
 * separate pass. Each exchange wait is bounded: one that gives up (which a
 * cooperative launch rules out) is counted, and dn_wait_give_ups() reports
 * the count. fwd.workspace, if given, holds
 * dn_chunk_fwd_out_norm_workspace_bytes(). */
typedef struct {
  dn_chunk_fwd_args fwd;
  const void *gate;       /* NULL for OutNorm::Plain */
  int64_t gate_stride;    /* elements between consecutive tokens' gate rows */
  int32_t gate_dtype;     /* DN_F32 or DN_BF16 */
  const float *weight;    /* gamma [head_v_dim] */
  double eps;
  int32_t in_scan;        /* 0: a separate norm pass; 1: the norm in the scan's y write */
} dn_chunk_fwd_out_norm_args;

int dn_chunk_fwd_out_norm(const dn_chunk_fwd_out_norm_args *args, hipStream_t stream);
size_t dn_chunk_fwd_out_norm_workspace_bytes(const dn_chunk_fwd_out_norm_args *args);

/* QkvProjection::forward (src/common/qkv.rs:373-449) and then
 * DeltaChunkBackendExt::delta_chunk_recalculated (chunk_recalculated.rs:115-151)
 * on its outputs, as every family runs them over a sequence
 * (gated_deltanet_1.rs:162-177, deltanet.rs:151-165, gated_deltanet_2.rs:213-261).
 * `fe` as for dn_frontend (n_householder 1); `fwd` as for dn_chunk_fwd, with
 * fwd.q, k, v, erase and write the front-end's outputs fe.q, k, v, erase and
 * write (the same pointers), and the sizes, gate widths and q/k/v dtype that
 * follow from fe. The results, the front-end's outputs and the next conv
 * window included, are those of dn_frontend followed by dn_chunk_fwd, bit for
 * bit. Where the chunk forward runs the two-kernel MFMA path with per-head
 * gates at head_k_dim 128, with a conv of length 4 and SiLU as the conv's and
 * the q/k activation (the reference's default), a bf16 projection, window and
 * q/k/v, 16-byte aligned rows and no check_finite, the front-end's q/k
 * half runs in the chunk forward's load stage: its intra kernel reads the raw
 * projection columns and the conv window, applies the conv, the activations
 * and the L2 norm, and writes q and k for the scan, so the projection's q/k
 * columns are read once and q and k written once, where the two calls write
 * them and read them twice. Otherwise the call runs the two calls. The
 * workspace is dn_chunk_fwd's (dn_frontend_chunk_fwd_workspace_bytes). */
typedef struct {
  dn_frontend_args fe;
  dn_chunk_fwd_args fwd;
} dn_frontend_chunk_fwd_args;

int dn_frontend_chunk_fwd(const dn_frontend_chunk_fwd_args *args, hipStream_t stream);
size_t dn_frontend_chunk_fwd_workspace_bytes(const dn_frontend_chunk_fwd_args *args);

/* Bounded cross-workgroup waits that gave up on the current device since the
 * library was loaded (synchronises the device). No counterpart in the
 * reference; nonzero means an output of dn_chunk_fwd_out_norm was wrong. */
int64_t dn_wait_give_ups(void);

/* One decode token of a delta-rule block between its in_proj and out_proj
 * GEMMs, in one launch: QkvProjection::step (src/common/qkv.rs:454-516: the
 * short-convolution step with its rolling window, the activations, the q/k
 * L2 norm, the write gates), delta_step (src/delta/recurrent.rs:41-99) on the
 * state, and OutNorm::forward (src/common/norm.rs:127-134): what a Gated
 * DeltaNet block's step (gated_deltanet_1.rs:218-234) runs there, given its
 * forget gate. Same fields and meaning as dn_frontend (sequence 1), dn_step
 * and dn_out_norm, whose composition it equals, with q, k, v and y kept in
 * fp32 between the stages. The output norm's gate, when present, is the
 * projection's segment after the write gates (qkv.rs:237-262), read in place.
 * One workgroup owns a (batch, head): n_householder = 1, head_k_dim and
 * head_v_dim up to DN_BLOCK_STEP_MAX_HEAD_DIM; other shapes return
 * DN_ERR_UNSUPPORTED (the three separate calls cover them). */
#define DN_BLOCK_STEP_MAX_HEAD_DIM 256
typedef struct {
  int64_t batch, nheads, head_k_dim, head_v_dim;
  int64_t conv_kernel;          /* 0: no short convolution; else 1..DN_FRONTEND_MAX_KERNEL */
  int64_t proj_stride;          /* elements from one batch row of the projection to the next */
  int32_t conv_activation;      /* DN_ACT_SILU or DN_ACT_IDENTITY */
  int32_t qk_activation;        /* dn_activation */
  int32_t qk_norm;              /* DN_QKNORM_L2 or DN_QKNORM_NONE */
  int32_t write_gate;           /* dn_write_gate */
  int32_t allow_neg_eigval;
  int32_t in_dtype;             /* projected and the windows: DN_F32 or DN_BF16 */
  int32_t out_dtype;            /* out: DN_F32 or DN_BF16 */
  int32_t has_gate;             /* forget gate present */
  int64_t decay_width;          /* 1 or head_k_dim, read when has_gate */
  double scale;                 /* NaN => 1/sqrt(head_k_dim) */
  double eps;                   /* the output norm's epsilon */
  int32_t norm_gated;           /* OutNorm::Gated (the gate segment follows the write gates) */
  int32_t check_finite;
  const void *projected;        /* [batch, proj_stride] */
  const float *conv_weight;     /* [conv_dim, conv_kernel] */
  const float *conv_bias;       /* [conv_dim] or NULL */
  const void *window_in;        /* [batch, conv_dim, conv_kernel], newest column last */
  void *window_out;             /* same shape; may alias window_in */
  const float *g;               /* [batch, nheads, decay_width] log forget gate */
  const float *state_in;        /* [batch, nheads, head_k_dim, head_v_dim] */
  float *state_out;             /* may alias state_in */
  const float *norm_weight;     /* gamma [head_v_dim] */
  void *out;                    /* [batch, nheads, head_v_dim] */
  float *y;                     /* optional [batch, nheads, head_v_dim]: the output before the norm */
} dn_block_step_args;

int dn_block_step(const dn_block_step_args *args, hipStream_t stream);

/* How unit_lower_inverse inverts I − N (TriSolve, src/delta/tri.rs:53-64). */
typedef enum {
  DN_TRI_BLOCKED = 0, /* the exact inverse without powers of N (the default) */
  DN_TRI_NEUMANN = 1, /* the series I + N + … + N^{size−1}, term by term in fp32 */
} dn_tri_solve;

/* Largest `size` DN_TRI_NEUMANN serves (N and the running term in LDS). The
 * reference keeps the series as a test baseline, usable to L ≈ 16
 * (tri.rs:59-63). */
#define DN_TRI_NEUMANN_MAX_SIZE 140

typedef struct {
  int64_t batch;          /* matrices: the product of the leading axes (≥ 0) */
  int64_t size;           /* the square trailing block (≥ 0) */
  int32_t solve;          /* dn_tri_solve */
  int32_t check_finite;   /* the reference's sanity check of input and output */
  const float *n_strict;  /* [batch, size, size] float32, strictly lower triangular */
  float *t;               /* [batch, size, size] float32; must not alias n_strict */
} dn_tri_args;

/* Replaces unit_lower_inverse (src/delta/tri.rs:66-114): T = (I − N)⁻¹ for a
 * batched strictly lower triangular N. As in the reference the caller owes the
 * strict lower property: DN_TRI_BLOCKED reads only N's strict lower triangle,
 * DN_TRI_NEUMANN multiplies the whole matrix. The square-block assert
 * ("unit_lower_inverse expects a square trailing block") belongs to the
 * caller, which passes one `size`. */
int dn_unit_lower_inverse(const dn_tri_args *args, hipStream_t stream);

/* Bytes of device workspace dn_chunk_fwd / dn_chunk_bwd need for these
 * arguments (0 on invalid arguments). Has no counterpart in the reference,
 * whose tensors are allocated by Burn; it lets a caller own the memory.
 *
 * A caller that passes workspace = NULL gets the library-managed workspace:
 * one grow-only buffer per device. It is meant for a single stream: calls on
 * two streams of one device at once share it and race. Growing it allocates
 * with hipMalloc and drains the device first (hipDeviceSynchronize), so the
 * first call at a new largest size is not asynchronous; under HIP graph
 * capture growth is refused (DN_ERR_HIP, hipErrorStreamCaptureUnsupported).
 * Callers that capture graphs, use several streams, or must not allocate in
 * the call pass their own workspace of at least these many bytes. */
size_t dn_chunk_fwd_workspace_bytes(const dn_chunk_fwd_args *args);
size_t dn_chunk_bwd_workspace_bytes(const dn_chunk_bwd_args *args);

/* dn_chunk_fwd for callers that cannot allocate: code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc. No counterpart in the
 * reference, whose Burn backend allocates every tensor. It takes the same
 * arguments and gives the same results as dn_chunk_fwd, but ignores
 * `workspace` and runs on a fixed scratch array of DN_NOALLOC_SCRATCH_BYTES
 * that the library holds on each device it runs on until the process ends
 * (the array is part of the loaded code object). It calls no hipMalloc,
 * hipFree or other allocating routine. Limits:
 *   - arguments whose dn_chunk_fwd_workspace_bytes() exceeds
 *     DN_NOALLOC_SCRATCH_BYTES return DN_ERR_WORKSPACE (the MFMA path needs
 *     24.25 KiB per (batch, head, chunk of 64 tokens) with per-head gates,
 *     so 64 MiB covers 2700 of them, e.g. batch 1 x 16 heads x 10,700
 *     tokens);
 *   - check_finite is refused (DN_ERR_UNSUPPORTED): the guard allocates its
 *     flag and synchronises;
 *   - every call on one device shares that device's array, so calls that
 *     overlap on one device (two streams, or two host threads) race; the
 *     array keeps the last call's contents, and no kernel reads any of it
 *     before writing it. */
#define DN_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int dn_chunk_fwd_noalloc(const dn_chunk_fwd_args *args, hipStream_t stream);

/* The algorithm a call runs (DN_ALGO_GENERIC, DN_ALGO_MFMA or, for the
 * forward, DN_ALGO_MFMA_FUSED), or DN_ERR_UNSUPPORTED for a requested MFMA
 * path that does not cover the arguments. */
int dn_chunk_fwd_algo(const dn_chunk_fwd_args *args);
int dn_chunk_bwd_algo(const dn_chunk_bwd_args *args);

/* Diagnostics; no counterpart in the reference, whose benches time whole calls
 * (benches/layer.rs:161-181). While profiling is on, every kernel the library
 * launches is bracketed by HIP events recorded on its own stream.
 * dn_profile_enable(1) clears earlier records. dn_profile_read synchronises on
 * the pending events and reports entry `index` (summed milliseconds and launch
 * count of one kernel name); it returns the number of entries. */
int dn_profile_enable(int on);
int dn_profile_read(int index, char *name, size_t name_len, double *total_ms,
                    int64_t *launches);

/* Text of the last error on this thread (empty string if none). */
const char *dn_last_error(void);

/* Library version string. */
const char *dn_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DELTANET_CORE_H */
