/*
 * dsalt_hip.h - C ABI of the gfx950 (MI355X) DSALT sparse-attention library
 * (libdsalt_hip.so).
 *
 * DSALT attention: query i of a packed sequence attends to its causal local window
 * plus k content-selected landmark tokens of its sequence. Two semantics exist:
 *
 *   HARD (inference):  band  j in [i - w(i) + 1, i],  w(i) = max(1, trunc(w[i]))
 *                      landmark p admitted iff 0 <= p <= i - w(i); logit bias lmk_bias[slot]
 *   SOFT (training):   band  0 <= d = i - j <= w~(i)  (fp32 compare), logit bias 0 in the
 *                      core d <= w~ - win_edge, log sigmoid((w~ - d) / tau_win) on the edge;
 *                      landmark p admitted iff p <= i and (float)p < (float)i - w~(i);
 *                      logit bias lmk_logw[slot]
 *   DENSE (batched):   one unpacked sequence [1, T, d]; every causal key j <= i of query i:
 *                      window bias 0 in the core d = i - j <= w~(i) - win_edge (fp32
 *                      compare), else log(max(sigmoid((w~(i) - d) / tau_win), 1e-20));
 *                      landmark bias lmk_bias[h, j] (an [H, T] table, -inf off the head's
 *                      landmarks) where d >= max(1, floor(w~(i))); the logit bias is the
 *                      larger of the two (equal biases share the gradient in halves)
 *
 * Logits are q.k * scale (+ bias); softmax is computed online in fp32; O is stored in
 * the input dtype and LSE = max + log(sum) in fp32 (natural log; -inf for empty rows,
 * whose O is 0).
 *
 * Conventions shared by every entry point:
 *   - All tensors are device pointers on the current HIP device. Packed token-major
 *     tensors are [T, H, D] with unit stride along D; strides are given in ELEMENTS.
 *   - Landmark positions are int64 [H, S, k], relative to the sequence start; -1 (or any
 *     value outside [0, L_s)) marks an empty slot.
 *   - cu_seqlens is int32 [S + 1], non-decreasing, cu_seqlens[0] = 0, cu_seqlens[S] = T.
 *     It lives on the device, so the host-side checks cannot read it; the kernels take
 *     sequence s as rows [clamp(cu[s], 0, T), max(clamp(cu[s+1], 0, T), that start)), so
 *     that no content of cu_seqlens makes them read or write outside the T rows (a packing
 *     that breaks the rule above gives results for those clamped sequences, and RoPE gives
 *     NaN to a token before cu_seqlens[0]).
 *   - `stream` is a hipStream_t (NULL = default stream). Calls are asynchronous on that
 *     stream, never synchronise and never allocate memory; the backward takes its scratch
 *     memory from a caller-provided workspace.
 *   - Every function returns DSALT_OK (0) or an error code; dsalt_last_error() returns a
 *     thread-local message describing the most recent failure on the calling thread.
 *   - Argument validation is host-side only (no device reads), so it also runs on a
 *     machine without a GPU (the *_check functions).
 */
#ifndef DSALT_HIP_H
#define DSALT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSALT_ABI_VERSION 3

enum {
    DSALT_OK = 0,
    DSALT_ERR_INVALID = 1,     /* bad argument (shape, stride, alignment, null pointer) */
    DSALT_ERR_UNSUPPORTED = 2, /* valid request this build does not support (e.g. D=96) */
    DSALT_ERR_LAUNCH = 3,      /* the HIP runtime rejected a kernel launch */
};

enum { DSALT_DTYPE_BF16 = 0, DSALT_DTYPE_F16 = 1, DSALT_DTYPE_F32 = 2 /* outputs and gradients only */ };
enum { DSALT_MODE_HARD = 0, DSALT_MODE_SOFT = 1, DSALT_MODE_DENSE = 2 };

/* Largest k_lmk the kernels accept (landmark slots per head and sequence). */
#define DSALT_MAX_K_LMK 1024

/*
 * Fused sparse-attention forward.
 * Replaces the Triton launches of
 *   _dsalt_fwd_kernel  (dsalt/kernels/dsalt_triton_attn.py:27-169, launched at :184-209)
 *   _train_fwd_kernel  (dsalt/kernels/dsalt_triton_train.py:74-214, launched at :629-645)
 * The landmark K/V gather of _build_landmark_kv (dsalt/kernels/selectors.py:137-159) and
 * the packed block map of _build_seq_block_map (selectors.py:37-67) happen inside the
 * kernel; `out` is written (no prior memset) in the input dtype, or in fp32 when
 * out_dtype = DSALT_DTYPE_F32 (the reference's entry points return O as fp32).
 * Limits: `scale` finite and non-zero (a negative scale is applied by negating Q);
 * (total_len + 64) x max(k, v row stride) x 2 bytes < 4 GiB (K/V rows of a sequence are
 * addressed with 32-bit offsets). Both are checked and return DSALT_ERR_UNSUPPORTED.
 *
 * DSALT_MODE_DENSE replaces the dense softmax of DSALTAttention._batched
 * (dsalt/modules/dsalt_attention.py:371-401, biases :286-329): num_seqs = 1, k_lmk = 0,
 * lmk_pos NULL, cu_seqlens may be NULL; lmk_bias is the [H, T] table lmk_bias[h, j] at
 * lmk_bias + h * lmk_bias_stride_h + j * lmk_bias_stride_k (NULL: no landmarks;
 * lmk_bias_stride_s is ignored); w holds w~; scale must be > 0.
 */
typedef struct dsalt_fwd_args {
    int32_t mode;      /* DSALT_MODE_HARD, DSALT_MODE_SOFT or DSALT_MODE_DENSE */
    int32_t dtype;     /* DSALT_DTYPE_* of q, k, v and out */
    int32_t total_len; /* T */
    int32_t num_seqs;  /* S >= 1 */
    int32_t n_heads;   /* H >= 1 */
    int32_t head_dim;  /* D, 64 or 128 */
    int32_t k_lmk;     /* landmark slots per (head, sequence), 0..DSALT_MAX_K_LMK */
    int32_t out_dtype; /* element type of out: `dtype` or DSALT_DTYPE_F32 */
    const void *q;
    int64_t q_stride_t, q_stride_h;
    const void *k;
    int64_t k_stride_t, k_stride_h;
    const void *v;
    int64_t v_stride_t, v_stride_h;
    void *out;
    int64_t out_stride_t, out_stride_h;
    float *lse; /* [T, H] fp32 */
    int64_t lse_stride_t, lse_stride_h;
    const float *w; /* [T]: HARD window sizes, SOFT continuous windows w~ */
    int64_t w_stride;
    const int64_t *lmk_pos; /* [H, S, k]; may be NULL when k_lmk == 0 */
    int64_t lmk_pos_stride_h, lmk_pos_stride_s, lmk_pos_stride_k;
    const float *lmk_bias; /* [H, S, k] fp32 (HARD lmk_bias, SOFT lmk_logw); NULL = 0 */
    int64_t lmk_bias_stride_h, lmk_bias_stride_s, lmk_bias_stride_k;
    const int32_t *cu_seqlens; /* [S + 1] */
    float scale;               /* logit scale, normally 1/sqrt(D) */
    float tau_win;             /* SOFT only */
    float win_edge;            /* SOFT only */
    int32_t n_kv_heads;        /* K/V heads, 0 = n_heads; must divide n_heads: query head h
                                  reads K/V head h / (n_heads / n_kv_heads) (grouped-query
                                  attention without a repeated K/V copy) */
    /* Optional RoPE of Q on load (HARD / SOFT): when rope_cos is not NULL, q holds the
     * un-rotated queries and the kernel rotates them as dsalt_rope would (half-split
     * pairs, the row of the query's position inside its sequence from rope_cos /
     * rope_sin [rope_rows, >= head_dim] fp32, rounded to the element type; NaN for a
     * position past the table). K must already be rotated. */
    const float *rope_cos, *rope_sin;
    int64_t rope_stride; /* row stride of the tables (elements) */
    int32_t rope_rows;
    int32_t rope_half;   /* 1: every row's columns D/2.. equal its columns ..D/2 (tables built
                            as cat(freqs, freqs)); the kernel then reads half of each row */
} dsalt_fwd_args;

int dsalt_fwd(const dsalt_fwd_args *args, void *stream);
/* Validation of dsalt_fwd's arguments without launching anything. */
int dsalt_fwd_check(const dsalt_fwd_args *args);

/*
 * Sparse-attention backward (both modes): dQ, dK, dV, the landmark-bias gradient and,
 * in SOFT mode, the gradient with respect to the continuous window (summed over heads).
 * Replaces
 *   _train_bwd_preprocess / _train_bwd_dkdv_kernel / _train_bwd_kernel
 *       (dsalt/kernels/dsalt_triton_train.py:220-481, launched at :693-745) and the
 *       d_w.sum(1) of :748
 *   dsalt_triton_backward (dsalt/kernels/dsalt_triton_bwd.py:219-324) with its kernels
 *       _dsalt_bwd_preprocess / _dsalt_bwd_kernel (:17-216).
 * Deterministic: no atomics; every output element is written by exactly one thread.
 * DSALT_MODE_DENSE (the autograd backward of the dense softmax of DSALTAttention._batched,
 * dsalt/modules/dsalt_attention.py:371-401): the forward's conventions; d_lmk_bias is
 * [H, T] contiguous (the gradient of every lmk_bias[h, j], 0 where it is -inf) and d_w is
 * [T]. dsalt_bwd_workspace_size(T, 1, H, D, 0) covers its workspace.
 */
typedef struct dsalt_bwd_args {
    int32_t mode, dtype, total_len, num_seqs, n_heads, head_dim, k_lmk;
    int32_t grad_dtype; /* dq/dk/dv element type: `dtype` or DSALT_DTYPE_F32 */
    int32_t out_dtype;  /* element type of the saved forward output: `dtype` or DSALT_DTYPE_F32 */
    int32_t n_kv_heads; /* as in dsalt_fwd_args; dk/dv are still per query head [T, H, D]
                           (the caller sums each group of n_heads / n_kv_heads heads) */
    const void *q;
    int64_t q_stride_t, q_stride_h;
    const void *k;
    int64_t k_stride_t, k_stride_h;
    const void *v;
    int64_t v_stride_t, v_stride_h;
    const void *out; /* forward output [T, H, D] in out_dtype */
    int64_t out_stride_t, out_stride_h;
    const float *lse; /* forward LSE [T, H] */
    int64_t lse_stride_t, lse_stride_h;
    const void *dout; /* upstream gradient, input dtype */
    int64_t dout_stride_t, dout_stride_h;
    const float *w;
    int64_t w_stride;
    const int64_t *lmk_pos;
    int64_t lmk_pos_stride_h, lmk_pos_stride_s, lmk_pos_stride_k;
    const float *lmk_bias;
    int64_t lmk_bias_stride_h, lmk_bias_stride_s, lmk_bias_stride_k;
    const int32_t *cu_seqlens;
    void *dq; /* [T, H, D] in grad_dtype */
    int64_t dq_stride_t, dq_stride_h;
    void *dk;
    int64_t dk_stride_t, dk_stride_h;
    void *dv;
    int64_t dv_stride_t, dv_stride_h;
    float *d_lmk_bias; /* [H, S, k] contiguous fp32; may be NULL */
    float *d_w;        /* [T] fp32, SOFT only; may be NULL */
    void *workspace;   /* >= dsalt_bwd_workspace_size(...) bytes, 256-byte aligned */
    int64_t workspace_bytes;
    float scale, tau_win, win_edge, reserved1;
} dsalt_bwd_args;

int64_t dsalt_bwd_workspace_size(int32_t total_len, int32_t num_seqs, int32_t n_heads,
                                 int32_t head_dim, int32_t k_lmk);
int dsalt_bwd(const dsalt_bwd_args *args, void *stream);
int dsalt_bwd_check(const dsalt_bwd_args *args);

/*
 * dsalt_bwd without a caller workspace and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The backward's scratch (per-query records, block band starts, per-head window
 * partials, landmark partials) lives in a static device array of
 * DSALT_NOALLOC_SCRATCH_BYTES bytes that the library holds on every GPU it runs on until
 * the process ends; args->workspace and args->workspace_bytes are ignored. A call whose
 * dsalt_bwd_workspace_size(...) exceeds that size returns DSALT_ERR_UNSUPPORTED without
 * launching. Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (other streams, other threads) race and must be serialised by the caller. The array
 * keeps the last call's contents; the kernels write every scratch entry they read.
 * The first call on a device looks the array's address up (with that device current).
 * The size covers the backward of every benchmark configuration of the reference (the
 * largest, 16 heads x 128 dims over one 16384-token sequence with k = 128, needs 75.3 MiB);
 * since the array sits in the library's code object, every process that loads the
 * library holds it on each GPU it launches on, whether or not it calls this entry point.
 */
#define DSALT_NOALLOC_SCRATCH_BYTES ((int64_t)76 << 20)
int dsalt_bwd_noalloc(const dsalt_bwd_args *args, void *stream);

/*
 * Landmark top-k selection.
 * Replaces the covered mask, the per-(head, sequence) torch.topk and the -1 fill of
 * _compute_landmark_indices (dsalt/kernels/selectors.py:105-134).
 * Token j at offset o inside its sequence is a candidate iff o >= trunc(w[j]). For each
 * (head, sequence) the min(k, L) largest scores are taken (NaN ranks above +inf, which
 * ranks above every finite score; equal scores: the lower position wins). Selected
 * finite-score positions are written in ascending order, followed by -1 in every
 * remaining slot (the reference's -inf/NaN/+inf slots also become -1).
 * workspace (optional, NULL allowed): with at least dsalt_select_workspace_size(...)
 * bytes, sequences longer than 4096 tokens (with ceil(L / 2048) * (k + min(k, 128)) <=
 * 8192) are selected in two stages - a superset of the top k of every 2048-position chunk
 * (at most k + min(k, 128) candidates) by one workgroup each, then the top k of the chunks'
 * candidates - instead of by one workgroup per (head, sequence). The result is identical; the workspace only adds parallelism. A size of 0
 * means no sequence can use it. max_seqlen: 0, or a bound on every sequence's length
 * (the chunk stage is skipped when it is <= 4096, saving its launch when no sequence is
 * long; a bound that is too small only means the one-workgroup route for everything).
 * w_out (optional, NULL allowed): fuses the window quantisation of
 * DSALTAttention._window_sizes(floor=True) (dsalt/modules/dsalt_attention.py:277-284)
 * into the selection. w then holds the continuous windows w~; w_out [T] (contiguous)
 * receives q(w~) = max(1, floor(w~)) (NaN stays NaN) for every token of
 * [cu_seqlens[0], cu_seqlens[S]), and a token is covered iff o + 1 <= q(w~) - the
 * selection is that of dsalt_quantize_windows followed by this call without w_out.
 * w_out may equal w (in place).
 * w_logit (optional, NULL allowed; needs w_out): the window gate's logits [T] (the
 * win_gate output of DSALTAttention._window_continuous, dsalt/modules/dsalt_attention.py:
 * 270-276) in w_logit_dtype. The windows are then computed in the launch as the module
 * computes them, w~ = n_min + sigmoid(logit) * (n_max - n_min), with every intermediate
 * (the sigmoid 1 / (1 + exp(-x)) in fp32, the product, the sum) rounded to w_logit_dtype
 * as torch's 16-bit elementwise ops round them - bit for bit torch's windows for every
 * bf16 and fp16 logit value; w is not read (may be NULL) and w_out receives q(w~) as
 * above. fp32 logits are not taken (DSALT_ERR_UNSUPPORTED): torch's fp32 sigmoid can
 * differ from this formula in the last bit.
 */
typedef struct dsalt_select_args {
    int32_t total_len, num_seqs, n_heads, k_lmk;
    const float *scores; /* [T, H] fp32 */
    int64_t scores_stride_t, scores_stride_h;
    const float *w; /* [T] window sizes */
    int64_t w_stride;
    const int32_t *cu_seqlens;
    int64_t *lmk_pos; /* out: [H, S, k] contiguous int64 */
    void *workspace;  /* NULL, or >= dsalt_select_workspace_size(...) bytes, 16-byte aligned */
    int64_t workspace_bytes;
    int32_t max_seqlen; /* 0 (unknown) or an upper bound on the sequence lengths */
    float *w_out;       /* NULL, or [T] fp32: quantised windows (w is then w~) */
    const void *w_logit;    /* NULL, or [T] window-gate logits (then w is not read) */
    int64_t w_logit_stride;
    int32_t w_logit_dtype;  /* DSALT_DTYPE_BF16 or _F16 */
    float n_min, n_max;     /* the module's window bounds */
} dsalt_select_args;

int64_t dsalt_select_workspace_size(int32_t total_len, int32_t num_seqs, int32_t n_heads, int32_t k_lmk);
int dsalt_select_landmarks(const dsalt_select_args *args, void *stream);
int dsalt_select_check(const dsalt_select_args *args);

/*
 * Hybrid landmark scores from the value projection (fused selector front-end).
 * Replaces hybrid_scores_per_head (dsalt/kernels/landmark_tokens_ker.py:19-61) without
 * its x @ W_V^T GEMM: v is the pre-RoPE value projection x W_V^T [T, n_kv, D] that the
 * attention module computes anyway. For token t and query head h (kv group
 * g = h / (n_heads / n_kv_heads)):
 *   scores[t, h] = alpha[h] * z_v[t, h] + (1 - alpha[h]) * z_x[t]
 *   z_x[t] = (||x_t|| - mean) / max(std, 1e-6),  z_v[t, h] = the same over ||v_t,g||
 * with mean and unbiased std over all T tokens (NaN std kept, as torch's clamp does).
 * The norms are taken in fp32 and rounded to the input dtype, as x.norm() returns them
 * for a 16-bit tensor, unless norms_f32 is nonzero: torch's autocast computes .norm() in
 * fp32 and returns it unrounded. x, v: unit stride along d / D, 16-byte aligned rows; D / (16 bytes
 * / v's element size) must be a power of two <= 64; n_kv_heads <= 128 and divides n_heads.
 * The means and stds are reduced in fp64 in a fixed order: the result is deterministic.
 */
typedef struct dsalt_scores_args {
    int32_t total_len, d_model, n_kv_heads, head_dim, n_heads;
    int32_t x_dtype, v_dtype; /* each DSALT_DTYPE_BF16, _F16 or _F32 (autocast: fp32 x, bf16 v) */
    int32_t norms_f32;        /* nonzero: keep the norms in fp32 (.norm() under autocast) */
    const void *x; /* [T, d_model] */
    int64_t x_stride_t;
    const void *v; /* [T, n_kv_heads, head_dim] */
    int64_t v_stride_t, v_stride_h;
    const float *alpha; /* [n_heads] */
    float *scores;      /* out: [T, n_heads] */
    int64_t scores_stride_t, scores_stride_h;
    float *z_x; /* out: [T] contiguous, may be NULL */
    float *z_v; /* out: [T, n_heads], may be NULL */
    int64_t z_v_stride_t, z_v_stride_h;
    void *workspace; /* >= dsalt_scores_workspace_size(...) bytes, 256-byte aligned */
    int64_t workspace_bytes;
    /* Optional: the RoPE of k in the same pass (what dsalt_rope does for k alone, same
     * arithmetic and table rules): k [T, n_kv_heads, head_dim] in v_dtype, rotated into
     * k_out (may alias k); the rows of cos/sin are positions inside the sequence given by
     * cu_seqlens (NULL: token t reads row t). k = NULL: no rotation. */
    const void *k;
    int64_t k_stride_t, k_stride_h;
    void *k_out;
    int64_t k_out_stride_t, k_out_stride_h;
    const float *rope_cos, *rope_sin;
    int64_t rope_stride;
    int32_t rope_rows, num_seqs;
    const int32_t *cu_seqlens;
    /* Optional: the window gate's logit in the same pass, which replaces the GEMV of
     * DSALTAttention._window_continuous (win_gate(x), dsalt/modules/dsalt_attention.py:
     * 270-276): gate_out[t] = x_t . gate_w + gate_b[0], the products summed in fp32 in a
     * fixed order (per lane over its 16-byte chunks, then a butterfly over the 64 lanes),
     * the bias added, rounded once to x_dtype. 16-bit x only. gate_w [d_model] and gate_b
     * [1] in x_dtype, 16-byte aligned (gate_b may be NULL: no bias); gate_out [T]
     * contiguous in x_dtype, e.g. the w_logit of the selection that follows.
     * gate_w = NULL: no logit (gate_b and gate_out must then be NULL). */
    const void *gate_w, *gate_b;
    void *gate_out;
} dsalt_scores_args;

int64_t dsalt_scores_workspace_size(int32_t total_len, int32_t n_kv_heads);
int dsalt_hybrid_scores(const dsalt_scores_args *args, void *stream);
int dsalt_scores_check(const dsalt_scores_args *args);

/*
 * Landmark selection with the hybrid scores formed inside the selection launch.
 * Replaces, in one call, hybrid_scores_per_head (dsalt/kernels/landmark_tokens_ker.py:
 * 19-61) and the selection of _compute_landmark_indices (dsalt/kernels/selectors.py:
 * 105-134) as DSALTAttention._packed chains them (dsalt/modules/dsalt_attention.py:
 * 655-666): the result is that of dsalt_hybrid_scores followed by dsalt_select_landmarks
 * on its scores, bit for bit (the same norms, the same fp64 statistics in the same order,
 * the same fp32 standardisation), with two launches instead of four: the norms pass
 * (which also rotates k when scores->k is set), then the selection, whose workgroups
 * derive the statistics of their head and score each candidate as they read it.
 * scores: as for dsalt_hybrid_scores, except that scores, z_x and z_v must be NULL (no
 * scores are written) and alpha is always required; its workspace must stay untouched
 * until the selection has run (same stream). select: as for dsalt_select_landmarks,
 * except that select->scores is not read (may be NULL). total_len and n_heads must agree.
 */
int dsalt_select_hybrid(const dsalt_scores_args *scores, const dsalt_select_args *select, void *stream);

/*
 * Rotary position embedding of q and k (half-split convention) in one pass.
 * Replaces apply_rotary_emb (dsalt/kernels/window_utils.py:73-88) as called by
 * DSALTAttention._packed (dsalt/modules/dsalt_attention.py:570-585): cos/sin rows are
 * rounded to the tensor dtype (the module's cos.to(q.dtype)), products and sums are
 * fp32 (no FMA contraction) and each result is rounded once, as the reference's
 * compiled function computes it. transpose = 1 applies the transposed rotation (the
 * backward: q = gradient of the output, q_out = gradient of the input).
 * cos, sin: fp32 tables with rows of head_dim entries (row stride cos_sin_stride). With
 * cu_seqlens, token t of sequence s reads row t - cu_seqlens[s] (the table must hold
 * max_s L_s rows, where the reference's table lookup would fail, rows past table_rows give
 * NaN outputs); with cu_seqlens = NULL, row t. q_out / k_out may alias q / k.
 * head_dim must be even; unit stride along head_dim.
 */
typedef struct dsalt_rope_args {
    int32_t total_len, num_seqs, n_q_heads, n_k_heads, head_dim;
    int32_t dtype; /* of q, k and the outputs: BF16, F16 or F32 */
    int32_t transpose;
    int32_t table_rows; /* rows of cos / sin; a token whose row is past them gets NaN */
    const void *q;
    int64_t q_stride_t, q_stride_h;
    const void *k;
    int64_t k_stride_t, k_stride_h;
    void *q_out;
    int64_t q_out_stride_t, q_out_stride_h;
    void *k_out;
    int64_t k_out_stride_t, k_out_stride_h;
    const float *cos, *sin;
    int64_t cos_sin_stride;
    const int32_t *cu_seqlens; /* may be NULL */
} dsalt_rope_args;

int dsalt_rope(const dsalt_rope_args *args, void *stream);
int dsalt_rope_check(const dsalt_rope_args *args);

/*
 * Window quantisation w = max(1, floor(w~)) (NaN stays NaN), the floor/clamp of
 * DSALTAttention._window_sizes(floor=True) and of _train_selectors
 * (dsalt/modules/dsalt_attention.py:277-284, :471). Either output may be NULL; the
 * int32 output holds 1 for NaN inputs, as the kernels' own clamp does.
 */
int dsalt_quantize_windows(const float *w_cont, int64_t n, float *w_out, int32_t *w_int_out,
                           void *stream);

/*
 * Gated SwiGLU product of the LM's feed-forward blocks: out = silu(gate) * up over n
 * elements of one dtype (DSALT_DTYPE_BF16, _F16 or _F32).
 * Replaces F.silu(gate_proj(x)) * up_proj(x) of SwiGLUFFN.forward
 * (dsalt/modules/dsalt_transformer.py:20-21) in one pass, with torch's two roundings:
 * silu(g) = g / (1 + exp(-g)) in fp32 rounded to the dtype, then the product in fp32
 * rounded again (bit for bit the two torch ops). gate, up, out: contiguous, 16-byte
 * aligned; n a multiple of 8 (16-bit) or 4 (fp32), else DSALT_ERR_UNSUPPORTED.
 */
int dsalt_swiglu(const void *gate, const void *up, void *out, int64_t n, int32_t dtype, void *stream);

/*
 * Residual add and RMSNorm of the LM's pre-norm blocks in one pass, per row of d elements:
 * x_out = x + h (each sum in fp32 rounded to the dtype, as torch's add), then
 * y = (x_out * rstd) * weight with rstd = rsqrt(sum(x_out^2) / d + eps) in fp32, rounded
 * to the dtype. h = NULL: y = RMSNorm(x) alone (x_out not written, may be NULL).
 * Replaces x = x + x_attn / x = x + x_ffn followed by the next RMSENorm
 * (dsalt/modules/dsalt_transformer.py:81-84; RMSENorm.forward, dsalt/kernels/RMSENorm.py:
 * 21-23) and the LM's final norm (dsalt/model/dsalt_lm.py:273). The sum of squares runs in
 * this pass's fixed order, so an output can differ from F.rms_norm's in its last bit
 * (a few in 10^6 in the tests); x_out is torch's sum exactly.
 * dtype BF16 or F16 for x, h, x_out, y and weight [d]; rows contiguous with row stride d;
 * d a multiple of 8, at most 4096; 16-byte aligned pointers; x_out may alias x or h, y
 * may alias none of them.
 */
int dsalt_add_rms_norm(const void *x, const void *h, void *x_out, void *y, const void *weight, int64_t rows,
                       int32_t d, float eps, int32_t dtype, void *stream);

int dsalt_abi_version(void);
const char *dsalt_last_error(void);
/* sizeof of the argument structs as compiled into the library (ABI layout check). */
size_t dsalt_fwd_args_size(void);
size_t dsalt_bwd_args_size(void);
size_t dsalt_select_args_size(void);
size_t dsalt_scores_args_size(void);
size_t dsalt_rope_args_size(void);

#ifdef __cplusplus
}
#endif

#endif /* DSALT_HIP_H */
