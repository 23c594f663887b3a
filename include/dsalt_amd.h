/*
 * dsalt_amd.h - C ABI of the MI355X (gfx950) DSALT sparse-attention library.
 *
 * Operator: query i of a packed sequence attends to A(i) = W(i) U L(i), where
 *   W(i) = [i - w_i + 1, i]                     (causal adaptive window, w_i >= 1)
 *   L(i) = { p in landmark set : 0 <= p < i - w_i + 1 }
 * so a landmark inside the window is counted once (as a window key).  Landmark
 * sets are chosen per (head, sequence) ("global") or per (head, sequence, query
 * block of block_size rows) from earlier positions only ("block-causal").
 *
 * Conventions shared by every entry point:
 *  - All pointers are device pointers unless stated otherwise.  The caller owns
 *    and allocates every buffer, including the workspace whose size the
 *    matching *_workspace_bytes() function returns.  The library never
 *    allocates device memory and never synchronises the stream.
 *  - Work is enqueued on `stream` (a hipStream_t passed as void*; NULL is the
 *    default stream).  Calls are stateless and may be made from any host thread;
 *    two calls that share a workspace must be ordered by the caller.
 *  - Return value: 0 on success, otherwise a DSALT_ERR_* code; a readable
 *    message for the last error of the calling thread is in dsalt_last_error().
 *  - Token tensors are packed: row t of q/k/v/out/h is token t of the batch,
 *    sequences delimited by cu_seqlens[0..num_seqs] (int32, cu_seqlens[0] = 0).
 *    Strides are in elements; the innermost (head_dim / hidden) stride is 1.
 *  - Landmark indices are int32, sequence-relative, ascending, padded with -1
 *    at the end of each set.  Layout [n_heads, num_seqs, n_sets, k_lmk] with
 *    n_sets = 1 (global) or ceil(max_seqlen / block_size) (block-causal).
 */
#ifndef DSALT_AMD_H
#define DSALT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSALT_ABI_VERSION 3

/* element types of token tensors */
#define DSALT_DTYPE_F32  0
#define DSALT_DTYPE_BF16 1
#define DSALT_DTYPE_F16  2

/* landmark selection variants */
#define DSALT_SELECT_GLOBAL 0  /* one set per (head, sequence), whole-sequence scores   */
#define DSALT_SELECT_BLOCK  1  /* one set per (head, sequence, query block), prefix scores */

/* scope of the z-score statistics in the global variant */
#define DSALT_STATS_PACKED   0 /* mean/std over all packed tokens (reference library) */
#define DSALT_STATS_SEQUENCE 1 /* mean/std per sequence                                 */

/* error codes */
#define DSALT_OK              0
#define DSALT_ERR_INVALID     1  /* bad argument (shape, dtype, null pointer)        */
#define DSALT_ERR_UNSUPPORTED 2  /* valid but not implemented on this build          */
#define DSALT_ERR_WORKSPACE   3  /* workspace missing or smaller than required       */
#define DSALT_ERR_HIP         4  /* a HIP runtime call failed (message has details)  */

typedef void* dsalt_stream_t; /* hipStream_t */

/* Problem shape shared by selection, forward and backward. */
typedef struct dsalt_problem {
    int32_t total_len;   /* T, packed tokens                                         */
    int32_t num_seqs;    /* S                                                        */
    int32_t max_seqlen;  /* max over s of cu_seqlens[s+1]-cu_seqlens[s] (host value) */
    int32_t n_heads;     /* H query heads                                            */
    int32_t n_kv_heads;  /* key/value heads, divides H (GQA when < H)                */
    int32_t head_dim;    /* D: 64 or 128                                             */
    int32_t k_lmk;       /* landmark slots per set, 0..2048 (training variant: 0..512) */
    int32_t select_mode; /* DSALT_SELECT_*                                           */
    int32_t block_size;  /* query block of the block-causal variant (>= 1; when not a multiple
                            of 64 the forward stages every set a 64-row tile's rows use: at
                            most 2048 slots, sets x k_lmk)                                     */
    int32_t dtype;       /* DSALT_DTYPE_* of the token tensors                       */
} dsalt_problem;

/*
 * Landmark selection.  Replaces, as one stream-ordered call:
 *   hybrid_scores_per_head        dsalt/kernels/landmark_tokens_ker.py:19-61
 *   _compute_landmark_indices     dsalt/kernels/selectors.py:75-134
 *   block-causal _select          results/causal_landmark_check.py:82-113
 * Score of token j for head h (kv head g = h / (H / n_kv_heads)):
 *   s = alpha_h * z(|v_{j,g}|) + (1 - alpha_h) * z(|h_j|)
 * with norms rounded to `dtype`, z-statistics in fp64 (unbiased std clamped at
 * 1e-6), candidates j_rel >= w_j (the token's own window), top-k with ties
 * broken by the lower index.  `v` holds x W_V^T without bias (the value
 * vectors); `h` the hidden states x.
 */
typedef struct dsalt_select_args {
    dsalt_problem p;
    int32_t hidden;            /* columns of h, multiple of 16 bytes / element size */
    int32_t stats_scope;       /* DSALT_STATS_* (global variant only)               */
    const void* h;   int64_t h_stride_t;                      /* [T, hidden]        */
    const void* v;   int64_t v_stride_t;  int64_t v_stride_h; /* [T, n_kv, D]       */
    const float* alpha;        /* [H], the mixing weight in (0, 1)                  */
    const int32_t* w;          /* [T] window sizes as integers                      */
    const int32_t* cu_seqlens; /* [S+1]                                             */
    int32_t* lmk_idx;          /* out [H, S, n_sets, k_lmk]                         */
    float* z_x;                /* optional out [T]      (global variant)            */
    float* z_v;                /* optional out [T, n_kv] (global variant)           */
    float* scores;             /* optional out [T, H]    (global variant)           */
    void* workspace; size_t workspace_bytes;
    /* Optional (NULL: none): a buffer of dsalt_plan_bytes(&p) bytes that receives the
     * forward's row plan of these rows (from w and cu_seqlens), computed in the same
     * launch as the norms.  dsalt_fwd with the same buffer, w, cu_seqlens and shape and
     * plan_ready set then skips its own plan pass.  No counterpart in the reference. */
    void* plan;
} dsalt_select_args;

/* Attention forward.  Replaces _dsalt_fwd_kernel and its launcher
 * dsalt/kernels/dsalt_triton_attn.py:27-169,184-209,259-311 (O and LSE).
 * out: [T, H, D] in dtype; lse: [T, H] fp32 natural-log sum of exponentials of
 * the scaled logits over A(i).  k/v may have n_kv_heads < n_heads (GQA). */
typedef struct dsalt_fwd_args {
    dsalt_problem p;
    const void* q;  int64_t q_stride_t; int64_t q_stride_h;
    const void* k;  int64_t k_stride_t; int64_t k_stride_h;
    const void* v;  int64_t v_stride_t; int64_t v_stride_h;
    const int32_t* w;          /* [T] window sizes (values < 1 act as 1)            */
    const int32_t* cu_seqlens; /* [S+1]                                             */
    const int32_t* lmk_idx;    /* [H, S, n_sets, k_lmk]                             */
    const float* lmk_bias;     /* [H, S, n_sets, k_lmk] added to landmark logits, or NULL */
    void* out;  int64_t o_stride_t; int64_t o_stride_h;
    float* lse;                /* [T, H] contiguous                                 */
    float scale;               /* logit scale, 1/sqrt(D) in the reference           */
    void* workspace; size_t workspace_bytes;
    /* Optional (NULL: none): a buffer of dsalt_plan_bytes(&p) bytes that receives
     * the row plan (per 64-row tile: rows ordered by window start, 16-row group
     * bounds, largest window) so dsalt_bwd of the same w / cu_seqlens / shape can
     * reuse it instead of recomputing it. */
    void* plan;
    /* Tile variant (DSALT_VARIANT_*; 0 = the library's default for the shape).  The
     * variants compute the same result with different tilings; which is fastest
     * depends on the shape (the autotune of dsalt/kernels/autotune.py:55-238). */
    int32_t variant;
    /* Non-zero: `plan` already holds the row plan of this call's w, cu_seqlens and shape
     * (written by dsalt_select or an earlier dsalt_fwd) and is read, not recomputed.
     * Ignored without `plan`, and by dsalt_train_fwd (its windows are floor(w~) + 1). */
    int32_t plan_ready;
} dsalt_fwd_args;

/* Attention backward.  Replaces _dsalt_bwd_preprocess + _dsalt_bwd_kernel and
 * dsalt_triton_backward, dsalt/kernels/dsalt_triton_bwd.py:17-324.
 * Deterministic: no floating-point atomics.  dq/dk/dv are contiguous
 * in dtype with dq [T, H, D] and dk/dv [T, n_kv_heads, D] (grouped heads: each
 * key/value head's gradient sums its query heads in head order, inside the
 * kernels); d_bias (optional) is fp32 [H, S, n_sets, k_lmk].  Global selection
 * variant only. */
typedef struct dsalt_bwd_args {
    dsalt_problem p;
    const void* q;    int64_t q_stride_t;  int64_t q_stride_h;
    const void* k;    int64_t k_stride_t;  int64_t k_stride_h;
    const void* v;    int64_t v_stride_t;  int64_t v_stride_h;
    const void* out;  int64_t o_stride_t;  int64_t o_stride_h;
    const void* dout; int64_t do_stride_t; int64_t do_stride_h;
    const float* lse;          /* [T, H] from the forward                           */
    const int32_t* w;
    const int32_t* cu_seqlens;
    const int32_t* lmk_idx;
    const float* lmk_bias;     /* or NULL                                           */
    void* dq; void* dk; void* dv;
    float* d_bias;             /* or NULL                                           */
    float scale;
    void* workspace; size_t workspace_bytes;
    const void* plan;          /* or NULL: the row plan dsalt_fwd wrote for the same
                                  w / cu_seqlens / shape (dsalt_fwd_args.plan)      */
    int32_t variant;           /* DSALT_VARIANT_* (0 = default)                     */
} dsalt_bwd_args;

/* Landmark K/V gather.  Replaces _build_landmark_kv, dsalt/kernels/selectors.py:137-159:
 * lmk_k/lmk_v [H, S, n_sets, k_lmk, D] (dtype), rows of invalid (-1) slots zero. */
typedef struct dsalt_gather_args {
    dsalt_problem p;
    const void* k;  int64_t k_stride_t; int64_t k_stride_h;
    const void* v;  int64_t v_stride_t; int64_t v_stride_h;
    const int32_t* cu_seqlens;
    const int32_t* lmk_idx;
    void* lmk_k; void* lmk_v;
} dsalt_gather_args;

int    dsalt_abi_version(void);
const char* dsalt_last_error(void);

/* Training variant with differentiable selectors.  Replaces _train_fwd_kernel,
 * _train_bwd_kernel and _train_bwd_dkdv_kernel with their wrapper
 * DSALTTrainFunction (dsalt/kernels/dsalt_triton_train.py:74-216,241-490,586-762),
 * whose semantics are the dense log-bias of dsalt/modules/dsalt_attention.py:520-563:
 * band keys j with 0 <= i - j <= w~(i) (continuous window w_cont, values below 0 act
 * as 0) carry the logit bias log sigmoid((w~ - d) / tau_win) where d = i - j >
 * w~ - win_edge (0 in the core); landmarks p with p < i - w~ get lmk_bias (the
 * log-weight log sigmoid(s / tau_lmk), -inf for empty slots).  base.w is not read.
 * Global landmark sets only. */
typedef struct dsalt_train_fwd_args {
    dsalt_fwd_args base;       /* lmk_bias = landmark log-weights                    */
    const float* w_cont;       /* [T] continuous windows                             */
    float tau_win;             /* > 0                                                */
    float win_edge;            /* >= 0                                               */
} dsalt_train_fwd_args;

/* Backward of the training variant: dq, dk, dv, d_bias (= d lmk_logw) as
 * dsalt_bwd, plus d_w [T]: d loss / d w~ summed over heads (:708-757). */
typedef struct dsalt_train_bwd_args {
    dsalt_bwd_args base;
    const float* w_cont;
    float tau_win;
    float win_edge;
    float* d_w;                /* out [T]                                            */
} dsalt_train_bwd_args;

/* Rotary position embedding of the query and key heads, in place, e.g. on the
 * output of one fused QKV projection read through strides (the attention entry
 * points then read q, k and v from the same buffer).  Replaces the RoPE step of
 * DSALTAttention._packed, dsalt/modules/dsalt_attention.py:566-585 (cos/sin rows
 * gathered at each token's position in its sequence and cast to the tensor type,
 * q * cos + rotate_half(q) * sin with rotate_half(x) = [-x2, x1], x1/x2 the two
 * halves of the head; dsalt/kernels/window_utils.py apply_rotary_emb), with the
 * rounding of that expression evaluated one operation at a time in the tensor type.
 * Needs no workspace. */
typedef struct dsalt_rope_args {
    int32_t total_len;         /* T                                                  */
    int32_t num_seqs;          /* S                                                  */
    int32_t max_seqlen;        /* longest sequence (host value), <= max_pos          */
    int32_t n_q_heads;         /* heads rotated in q (may be 0)                      */
    int32_t n_k_heads;         /* heads rotated in k (may be 0)                      */
    int32_t head_dim;          /* multiple of 16, <= 256                             */
    int32_t dtype;             /* DSALT_DTYPE_*                                      */
    void* q; int64_t q_stride_t; int64_t q_stride_h;
    void* k; int64_t k_stride_t; int64_t k_stride_h;
    const int32_t* cu_seqlens;
    const float* cos;          /* [max_pos, head_dim] fp32, rows 16-byte aligned     */
    const float* sin;          /* [max_pos, head_dim]                                */
    int32_t max_pos;
} dsalt_rope_args;

int    dsalt_rope_qk(const dsalt_rope_args* a, dsalt_stream_t stream);

/* Attention probabilities of one sequence over the keys each row attends, in banded
 * form (O(L (w + k)) memory).  Replaces the dense [H, L, L] rebuild of _last_P for the
 * analysis metrics, dsalt/modules/dsalt_attention.py:636-702 (consumer
 * dsalt/training/trainer.py:88-135): p_win[h][i][c] = P(i, i - c) for window keys
 * c < min(w_i, i + 1) and 0 up to w_cap; p_lmk[h][i][slot] = P(i, landmark of the slot)
 * when the row sees it, else 0.  P = exp(scale * q_i . k_j + bias - lse_i) with the LSE
 * the forward returned, i.e. the probabilities the forward used (rows of the dense
 * matrix are the two parts scattered to their key columns).  Needs no workspace. */
typedef struct dsalt_probs_args {
    dsalt_problem p;
    const void* q;  int64_t q_stride_t; int64_t q_stride_h;
    const void* k;  int64_t k_stride_t; int64_t k_stride_h;
    const int32_t* w;
    const int32_t* cu_seqlens;
    const int32_t* lmk_idx;
    const float* lmk_bias;     /* or NULL                                           */
    const float* lse;          /* [T, n_heads] as returned by dsalt_fwd              */
    float scale;
    int32_t seq;               /* the exported sequence                             */
    int32_t rows;              /* rows of the outputs (its length)                  */
    int32_t w_cap;             /* columns of p_win, >= the largest window of its rows */
    float* p_win;              /* [n_heads, rows, w_cap]                             */
    float* p_lmk;              /* [n_heads, rows, k_lmk] or NULL                     */
} dsalt_probs_args;

int    dsalt_export_probs(const dsalt_probs_args* a, dsalt_stream_t stream);

/* Row cross-entropy of the fused linear cross-entropy: for each row of a chunk of logits
 * (x W^T of the LM head), the loss and, in place over the logits, the gradient of the
 * loss with respect to them.  Replaces liger_cross_entropy_kernel,
 * dsalt/kernels/cross_entropy.py:133-310 (ignore_index, class weights, label smoothing,
 * z-loss lse_square_scale * lse^2, softcap, reductions none/mean/sum, token accuracy and
 * predicted tokens), plus the token scaling of its driver (:420-446): every output of a
 * row times the row's probability of its target.  n_non_ignore / sum_non_ignore_weight /
 * weight_sum are the batch totals the "mean" reduction divides by.  Targets must be
 * ignore_index or in [0, n_cols); any n_cols >= 1; rows 16-byte aligned.  The
 * GEMMs around it (logits, grad_input, grad_weight) are the caller's. */
typedef struct dsalt_ce_args {
    int32_t rows;
    int32_t n_cols;            /* vocabulary size V                                  */
    int32_t dtype;             /* DSALT_DTYPE_* of the logits                        */
    void* logits; int64_t logits_stride;   /* [rows, V]; gradient written in place    */
    const int64_t* target;     /* [rows]                                             */
    const float* ce_weight;    /* [V] class weights or NULL                          */
    float* loss;               /* [rows] per-row loss (z-loss included)              */
    void* z_loss;              /* [rows] in the logits' type, or NULL                */
    float* accuracy;           /* [rows] 1 when the argmax is the target, or NULL    */
    int64_t* predicted;        /* [rows] argmax (first index), -1 for ignored rows   */
    int64_t ignore_index;
    float n_non_ignore;
    float sum_non_ignore_weight;
    float weight_sum;
    float lse_square_scale;
    float label_smoothing;
    float softcap;             /* 0: none                                            */
    int32_t reduction;         /* 0 none, 1 mean, 2 sum                              */
    int32_t want_grad;         /* write the gradient over the logits                 */
    int32_t token_scaling;
} dsalt_ce_args;

int    dsalt_cross_entropy_rows(const dsalt_ce_args* a, dsalt_stream_t stream);

/* Gated activation of the SwiGLU feed-forward block, out = silu(gate) * up, where
 * gate and up may be column ranges of one fused gate/up GEMM output.  Replaces
 * F.silu(gate_proj(x)) * up_proj(x) of SwiGLUFFN.forward,
 * dsalt/modules/dsalt_transformer.py:20-21 (silu in float32 as g / (1 + exp(-g))
 * rounded to the tensor type, the product rounded to the tensor type).  rows x cols
 * of any width; every row 16-byte aligned.  Needs no workspace. */
typedef struct dsalt_silu_mul_args {
    int32_t rows;
    int32_t cols;
    int32_t dtype;              /* DSALT_DTYPE_*                                     */
    const void* gate; int64_t gate_stride;   /* row strides in elements              */
    const void* up;   int64_t up_stride;
    void* out;        int64_t out_stride;
} dsalt_silu_mul_args;

int    dsalt_silu_mul(const dsalt_silu_mul_args* a, dsalt_stream_t stream);

/* Tile variants of the attention kernels (dsalt_fwd_args.variant, dsalt_bwd_args.variant).
 * Bits are independent; a bit a shape cannot use is ignored. */
#define DSALT_VARIANT_DEFAULT    0
#define DSALT_VARIANT_FWD_BN32   1  /* forward: 32-key chunks (16-bit types, head_dim 64)        */
#define DSALT_VARIANT_FWD_RG2    2  /* forward: two 16-row groups per wave (16-bit types)       */
#define DSALT_VARIANT_DQ_BN64    4  /* backward dQ: 64-key chunks (16-bit types, head_dim 64)     */
#define DSALT_VARIANT_LMK_SHORT  8  /* backward landmark pass: 512-row chunks                    */
#define DSALT_VARIANT_FWD_BN64  16  /* forward: 64-key chunks (16-bit types, head_dim 128,
                                       inference operator; ignored with FWD_RG2)                 */
#define DSALT_VARIANT_FWD_8W    32  /* forward: blocks of 128 rows, eight waves of one row group
                                       each (16-bit, head_dim 128, inference operator; ignores
                                       FWD_RG2 and FWD_BN64)                                     */
#define DSALT_VARIANT_MASK       63

/* Bytes of the row-plan buffer of dsalt_fwd_args.plan / dsalt_bwd_args.plan. */
size_t dsalt_plan_bytes(const dsalt_problem* p);

size_t dsalt_select_workspace_bytes(const dsalt_select_args* a);
int    dsalt_select(const dsalt_select_args* a, dsalt_stream_t stream);

/* Workspace of dsalt_fwd: the row plan, or 0 when a->plan supplies it. */
size_t dsalt_fwd_workspace_bytes(const dsalt_fwd_args* a);
int    dsalt_fwd(const dsalt_fwd_args* a, dsalt_stream_t stream);

/* dsalt_fwd without allocations or a workspace argument.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops on one stream, harnesses that forbid hipMalloc).  The
 * row plan goes to a file-scope device array of DSALT_FWD_NOALLOC_MAX_PLAN_BYTES per
 * GPU (held until the process ends) unless a->plan is given; a->workspace is not read.
 * Problems whose plan does not fit (dsalt_plan_bytes(&a->p) >
 * DSALT_FWD_NOALLOC_MAX_PLAN_BYTES: with its three 256-byte-aligned sections, more than
 * 31,772 tiles, where the tiles are num_seqs * ceil(max_seqlen / 64)) are rejected with
 * DSALT_ERR_WORKSPACE.
 * Single-stream contract: every call on one GPU shares that array, so calls without
 * a->plan must be ordered on one stream (or ordered by the caller across streams and
 * host threads).  Overlapping calls race on the array without any error being
 * reported.  Outputs are those of dsalt_fwd. */
#define DSALT_FWD_NOALLOC_MAX_PLAN_BYTES ((size_t)4 << 20)
int    dsalt_fwd_noalloc(const dsalt_fwd_args* a, dsalt_stream_t stream);

/* Workspace of dsalt_bwd (per-row data and landmark partials; the row plan too unless
 * a->plan supplies it). */
size_t dsalt_bwd_workspace_bytes(const dsalt_bwd_args* a);
int    dsalt_bwd(const dsalt_bwd_args* a, dsalt_stream_t stream);

int    dsalt_gather_landmarks(const dsalt_gather_args* a, dsalt_stream_t stream);

size_t dsalt_train_fwd_workspace_bytes(const dsalt_train_fwd_args* a);
int    dsalt_train_fwd(const dsalt_train_fwd_args* a, dsalt_stream_t stream);
size_t dsalt_train_bwd_workspace_bytes(const dsalt_train_bwd_args* a);
int    dsalt_train_bwd(const dsalt_train_bwd_args* a, dsalt_stream_t stream);

/* Testing hook with no counterpart in the reference: dsalt_select with its
 * top-k working sets shrunk by `border_cap` so tests can drive the paths that
 * large inputs and large tie groups take.  Block-causal sets: LDS capacity of
 * the radix boundary bin limited to `border_cap` keys (extra radix passes).
 * Global sets: candidates sorted per part and parts merged per merge block
 * limited by `border_cap` (many parts, several merge levels).  dsalt_select is
 * this call with the full capacity; the workspace it needs is
 * dsalt_select_workspace_bytes_cap(a, border_cap).  border_cap ==
 * DSALT_SELECT_FORCE_PRUNE is the full capacity with the block-causal candidate
 * pruning (bf16 inputs) run whatever the sequence length; dsalt_select runs it
 * for sequences of 65536 tokens or more. */
#define DSALT_SELECT_FORCE_PRUNE 0x3fffffff
int    dsalt_select_with_border_cap(const dsalt_select_args* a, dsalt_stream_t stream, int border_cap);
size_t dsalt_select_workspace_bytes_cap(const dsalt_select_args* a, int border_cap);

/* Per-kernel timing, an instrumentation facility with no counterpart in the
 * reference (its only timing is the CUDA-event fwd+bwd step of
 * dsalt/kernels/autotune.py:176-189).  While enabled, every kernel the library
 * enqueues is bracketed by two HIP events on its stream (events are created
 * once and reused).  dsalt_timing_report waits for the recorded events, writes
 * one line "kernel launches total_ms" per kernel name into buf (NUL-terminated,
 * truncated to len), resets the totals and returns the full report length. */
int    dsalt_timing_enable(int enable);
int    dsalt_timing_report(char* buf, size_t len);

#ifdef __cplusplus
}
#endif

#endif /* DSALT_AMD_H */
