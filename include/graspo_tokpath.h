/*
 * graspo_tokpath.h -- C ABI of the MI355X (gfx950) vocabulary-wide token path.
 *
 * Two operations, both HBM-bound streaming passes over [rows, V] logits:
 *
 *   1. gtp_sample_rows: the rollout sampler.  Per row: repetition penalty,
 *      allow-mask, temperature, top-k, top-p and an inverse-CDF draw from a
 *      caller-supplied uniform.  Bit-exact and deterministic: the draw uses
 *      fixed-point weights (see "Sampler contract" below), so the same inputs
 *      give the same ids on any device, in any reduction order.
 *   2. gtp_logprob_entropy_rows / gtp_lse_partial_rows: the per-token
 *      selective log-softmax gather and the softmax entropy, fp32 accumulation.
 *
 * Conventions shared by every entry point:
 *   - All array pointers are DEVICE pointers owned by the caller.  The library
 *     never allocates and is reentrant, with one exception:
 *     gtp_sample_rows_noalloc works in one library-owned array per GPU, so
 *     two of its calls that overlap on one GPU (different streams or host
 *     threads) race; the caller serialises them.  The library's only mutable
 *     global state is: the measurement hook's per-thread event pair
 *     (gtp_time_next_launch); a per-device cache of the compute-unit count,
 *     filled once per device with atomic stores; and that per-device array
 *     with its per-device address table.
 *   - Work is enqueued asynchronously on `stream` (a hipStream_t passed as
 *     void*; NULL is the default stream).
 *   - Return value: GTP_OK or a GTP_ERR_* code for a bad argument or a failed
 *     launch.  Data-dependent problems of a single row are reported per row
 *     through `out_status` (GTP_ROW_*), never through the return value.
 *   - Logits rows are `row_stride` elements apart (row_stride >= V), so a
 *     [B, S, V] tensor's last position can be passed without a copy.
 *
 * Sampler contract (per row; every step is one IEEE-754 fp32 operation):
 *   x_i   = float(logits[i])                         (bf16/fp16 -> fp32 is exact)
 *   status NONFINITE if any x_i is NaN or +inf; BAD_HISTORY if any history
 *   id >= V (ids < 0 are padding); BAD_UNIFORM unless 0 <= u < 1.
 *   x'_i  = i in set(history) ? (x_i < 0 ? x_i * rho : x_i / rho) : x_i
 *   allowed_i = mask == NULL || bit (i & 31) of mask[i >> 5] is set
 *   y_i   = T > 0 ? x'_i / max(T, 1e-6f) : x'_i
 *   valid = { i : allowed_i and y_i > -inf };  empty -> status EMPTY
 *   order = (y desc, id asc); NONFINITE if the largest y is +inf
 *   T <= 0 (greedy): id = first in order; kept = 1; sampled_logprob = 0.
 *          Greedy is torch's argmax (tensor_utils.py:658) over the allowed
 *          tokens' y: a NaN beats every value and +inf every finite one
 *          (first by id), and allowed tokens that are all -inf give the
 *          first of them.  Such rows are GTP_ROW_OK, with logprob NaN when
 *          the raw row holds a NaN or +inf; only no allowed token at all
 *          (EMPTY) or a bad history id fails a greedy row.
 *   top-k: if 0 < K < |valid| keep the first K, else keep all valid.
 *   m = y of the first in order; w_i = DETEXP_FIX(y_i - m) (uint64, 2^40 = 1.0)
 *   top-p: if 0 < P < 1, with W = sum of kept w and S_r = sum_{j<r} w_j,
 *          keep rank r iff S_r <= floor(P * W)  (first rank always kept).
 *   draw:  W' = sum of kept w; U = floor(u * W'); id = first rank r with
 *          S_{r+1} > U.
 *   outputs: id; kept = |kept set|; threshold (y, id) of the last kept rank;
 *            logprob = log_softmax(x)[id] (unpenalized, unmasked, T = 1);
 *            sampled_logprob = log(w_id / W').
 *   A row with status != OK gets id = -1, kept = 0, NaN logprobs.
 *
 * DETEXP_FIX(d) for d <= 0 (all fp32 except the last step):
 *   d < -30 -> 0;  n = rint(d * 0x1.715476p+0);
 *   r = fma(-n, 0x1.62e4p-1, d);  r = fma(-n, 0x1.7f7d1cp-20, r);
 *   p = Horner(r; 1/7! .. 1/2!, 1, 1) with fma, coefficients rounded to fp32;
 *   result = p * 2^(n + 40) rounded to an integer, ties to even.
 */
#ifndef GRASPO_TOKPATH_H
#define GRASPO_TOKPATH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type of the logits. */
enum gtp_dtype {
  GTP_DTYPE_F32 = 0,
  GTP_DTYPE_BF16 = 1,
  GTP_DTYPE_F16 = 2
};

/* Return codes. */
enum gtp_error {
  GTP_OK = 0,
  GTP_ERR_INVALID_ARGUMENT = 1,
  GTP_ERR_UNSUPPORTED = 2,
  GTP_ERR_LAUNCH = 3
};

/* Per-row status codes written to out_status. */
enum gtp_row_status {
  GTP_ROW_OK = 0,
  GTP_ROW_NONFINITE = 1,   /* NaN or +inf in the row (or +inf after temperature) */
  GTP_ROW_EMPTY = 2,       /* no allowed token with a finite processed logit */
  GTP_ROW_BAD_HISTORY = 3, /* a history id >= V */
  GTP_ROW_BAD_UNIFORM = 4, /* uniform outside [0, 1) */
  GTP_ROW_BAD_TARGET = 5   /* logprob target outside [0, V) */
};

/* Largest vocabulary the sampler handles (the per-row penalty bitmap and
 * candidate index live in LDS). */
#define GTP_SAMPLER_MAX_V (1 << 18)

typedef struct gtp_sampler_params {
  float temperature;        /* <= 0 selects greedy decoding */
  int32_t top_k;            /* 0 (or >= number of valid tokens) disables top-k */
  float top_p;              /* active iff 0 < top_p < 1 */
  float repetition_penalty; /* 1 disables; must be > 0 */
} gtp_sampler_params;

/*
 * gtp_sample_rows -- one sampled token per row.
 *
 * Replaces the reference's per-step sampler
 *   _next_token_from_logits  src/graspo/backends/graspoflow/tensor_utils.py:649-658
 *   _sample_next_token       src/graspo/backends/graspoflow/tensor_utils.py:671-683
 * (temperature, greedy argmax, softmax / sort / cumsum / top-p cut /
 * multinomial) and extends it with repetition penalty, allow-mask, top-k and
 * a supplied-uniform draw.
 *
 *   logits      [B, row_stride] of `dtype`, first V entries of each row used
 *   history     [B, hist_stride] int32, first hist_len used (NULL or
 *               hist_len == 0: no penalty)
 *   allow_mask  [B, mask_stride] uint32, mask_stride >= ceil(V/32), LSB-first
 *               (NULL: every token allowed)
 *   uniforms    [B] fp32 in [0, 1) (ignored for greedy rows; may be NULL then)
 *   finished    [B] uint8 or NULL; rows with finished[b] != 0 output
 *               pad_token_id as their id (the where() of
 *               _broadcast_and_pad_finished, tensor_utils.py:661-668)
 *   outputs     [B] each; any of them may be NULL except out_ids.
 *   workspace   device scratch of at least gtp_sample_workspace_bytes()
 *               bytes (may be NULL when that is 0), 256-byte aligned,
 *               zero-filled once when allocated.  Calls leave it ready for
 *               the next call; two calls that may run at the same time
 *               (e.g. on different streams) need different workspaces.
 */
int gtp_sample_rows(const void* logits, int dtype, int64_t B, int64_t V,
                    int64_t row_stride, const int32_t* history, int64_t hist_len,
                    int64_t hist_stride, const uint32_t* allow_mask,
                    int64_t mask_stride, const float* uniforms,
                    const gtp_sampler_params* params, const uint8_t* finished,
                    int64_t pad_token_id, int64_t* out_ids, float* out_logprob,
                    float* out_sampled_logprob, int32_t* out_kept,
                    float* out_thresh_value, int32_t* out_thresh_id,
                    int32_t* out_status, void* workspace, size_t workspace_bytes,
                    void* stream);

/*
 * gtp_sample_workspace_bytes -- workspace gtp_sample_rows needs for B rows of
 * V logits of `dtype` under `params` (0 when the call needs none).  Greedy and
 * top-k rows (1 <= top_k <= 128) split each row over several workgroups and
 * merge per-row candidate lists through the workspace.  bf16 top-p batches
 * (no top-k, V >= 65536) of up to 64 rows also split each row over several
 * workgroups, which merge their value counts through 64 KB slots (16.8 MB
 * for 64 rows of 151936); a smaller workspace gives them fewer slices, and
 * none one workgroup per row.  Other calls need none.
 */
size_t gtp_sample_workspace_bytes(int dtype, int64_t B, int64_t V,
                                  const gtp_sampler_params* params);

/*
 * gtp_sample_route -- which kernel gtp_sample_rows would run for a call, and
 * how many workgroups split each row; no counterpart in the reference (the
 * kernels are this library's).  For callers that choose an input format by
 * the kernel it reaches (the Python drop-in narrows fp32 rows to bf16 unless
 * the fp32 top-p kernel takes them) and for tests.
 *   aligned          nonzero when logits and row stride are 16-byte aligned
 *   hist_len         history entries per row (0: no history)
 *   has_mask         nonzero when an allow mask is passed
 *   workspace_bytes  the workspace the call would pass (0: none)
 * out_route gets one of GTP_ROUTE_*, out_slices the workgroups per row.
 */
#define GTP_ROUTE_SPLIT_TOPK 1  /* greedy / top-k <= 128: split sampler      */
#define GTP_ROUTE_TOPP_SPLIT 2  /* bf16 top-p rows of small batches, split   */
#define GTP_ROUTE_TOPP 3        /* bf16 top-p rows, one workgroup per row    */
#define GTP_ROUTE_TOPP32 4      /* fp32 top-p rows, one workgroup per row    */
#define GTP_ROUTE_HIST 5        /* bf16 value-histogram sampler              */
#define GTP_ROUTE_ROWWISE 6     /* row-wise sampler (every other call)       */
int gtp_sample_route(int dtype, int64_t B, int64_t V, int aligned, int64_t hist_len,
                     int has_mask, const gtp_sampler_params* params, size_t workspace_bytes,
                     int32_t* out_route, int32_t* out_slices);

/* Size of the library's own workspace for gtp_sample_rows_noalloc. */
#define GTP_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)

/*
 * gtp_sample_rows_noalloc -- gtp_sample_rows without a caller workspace and
 * without any allocation.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).
 *
 * Arguments and results are those of gtp_sample_rows (same kernels, same
 * bit-exact outputs).  The workspace is a device array of
 * GTP_NOALLOC_SCRATCH_BYTES inside the library, one per GPU, held until the
 * process ends; the first call on a device looks up that device's copy.
 * Each call that uses the array first clears its per-row counters with a
 * small fill kernel on `stream` (calls that need no workspace, such as
 * top-p rows on the one-workgroup kernels, use none).  bf16 top-p calls of small batches, whose split rows
 * would need more, split their rows over fewer workgroups (or none) to fit.
 * Returns GTP_ERR_UNSUPPORTED when any other call needs more than
 * GTP_NOALLOC_SCRATCH_BYTES (gtp_sample_workspace_bytes() tells), e.g.
 * thousands of fp32 rows of a 2^18 vocabulary.  Every call on one GPU shares
 * that GPU's array: calls that may overlap on one GPU (different streams,
 * host threads) race and must be serialised by the caller.
 */
int gtp_sample_rows_noalloc(const void* logits, int dtype, int64_t B, int64_t V,
                            int64_t row_stride, const int32_t* history, int64_t hist_len,
                            int64_t hist_stride, const uint32_t* allow_mask,
                            int64_t mask_stride, const float* uniforms,
                            const gtp_sampler_params* params, const uint8_t* finished,
                            int64_t pad_token_id, int64_t* out_ids, float* out_logprob,
                            float* out_sampled_logprob, int32_t* out_kept,
                            float* out_thresh_value, int32_t* out_thresh_id,
                            int32_t* out_status, void* stream);

/*
 * gtp_logprob_entropy_rows -- log_softmax(x)[target] and softmax entropy per
 * row, one streaming read of the row, fp32 accumulation.
 *
 * Replaces sequence_log_probs_from_logits  src/graspo/core/graspo_loss.py:19-21
 * (log_softmax over V, gather) without writing the [N, V] log-softmax; the
 * entropy -sum p log p has no reference counterpart.
 *
 *   targets      [N] int32 (targets_int64 == 0) or int64 token ids
 *   out_logprob  [N] fp32; out_entropy [N] fp32 or NULL; out_status [N] or NULL
 * A target outside [0, V) gives NaN logprob and GTP_ROW_BAD_TARGET.
 */
int gtp_logprob_entropy_rows(const void* logits, int dtype, int64_t N,
                             int64_t V, int64_t row_stride, const void* targets,
                             int targets_int64, float* out_logprob,
                             float* out_entropy, int32_t* out_status,
                             void* stream);

/*
 * gtp_lse_partial_rows -- fold one vocabulary chunk [col_offset, col_offset+Vc)
 * into a running per-row state (m, s, t, x_target), all fp32:
 *   m = running max, s = sum exp(x - m), t = sum exp(x - m) * (x - m),
 *   x_target = the target's logit once its chunk has been seen (else NaN).
 * accumulate == 0 starts a new state; != 0 merges into `state`.
 *
 * Replaces the vocabulary-chunk loop of _selected_token_log_probs_from_hidden
 * src/graspo/backends/graspoflow/tensor_utils.py:180-186 (logsumexp per chunk,
 * logaddexp across chunks); the chunk logits come from the caller's GEMM.
 */
int gtp_lse_partial_rows(const void* logits, int dtype, int64_t N, int64_t Vc,
                         int64_t row_stride, int64_t col_offset,
                         const void* targets, int targets_int64, float* state,
                         int accumulate, void* stream);

/* gtp_lse_finalize_rows -- logprob = x_target - m - log s and
 * entropy = log s - t / s from the state of gtp_lse_partial_rows. */
int gtp_lse_finalize_rows(const float* state, int64_t N, float* out_logprob,
                          float* out_entropy, void* stream);

/*
 * gtp_lm_head_logprob_rows -- logprob, entropy and logsumexp of the logits
 * x = h W^T per row without writing them: the bf16 lm_head GEMM runs on the
 * matrix cores (fp32 accumulation) with the online log-sum-exp in its
 * epilogue.
 *
 * Replaces _selected_token_log_probs_from_hidden
 * src/graspo/backends/graspoflow/tensor_utils.py:167-186 (index_select of
 * the target rows and their dot products, then F.linear + logsumexp +
 * logaddexp per vocabulary chunk) for operands that are bf16 values.
 *
 *   hidden   [N, K] bf16, rows hidden_stride elements apart
 *   weight   [V, K] bf16, rows weight_stride elements apart
 *   targets  [N] int32 (targets_int64 == 0) or int64 token ids
 *   out_logprob [N] = h_n . w_{t_n} - lse_n (the target logit is an fp32 dot
 *            product of the exact bf16 products, as the reference's
 *            selected_logits); out_entropy, out_lse [N] fp32 or NULL;
 *            out_status [N] or NULL.  A target outside [0, V) gives NaN
 *            logprob and GTP_ROW_BAD_TARGET.
 *   workspace of at least gtp_lm_head_workspace_bytes(N, V) bytes (partial
 *            states per vocabulary group; no contents carried between calls)
 * Returns GTP_ERR_UNSUPPORTED unless K is a multiple of 128, both pointers
 * are 16-byte aligned and both strides are multiples of 8 below 2^22.
 */
int gtp_lm_head_logprob_rows(const uint16_t* hidden, int64_t N, int64_t K,
                             int64_t hidden_stride, const uint16_t* weight, int64_t V,
                             int64_t weight_stride, const void* targets, int targets_int64,
                             float* out_logprob, float* out_entropy, float* out_lse,
                             int32_t* out_status, void* workspace, size_t workspace_bytes,
                             void* stream);
size_t gtp_lm_head_workspace_bytes(int64_t N, int64_t V);

/*
 * gtp_lm_head_logprob_save_rows -- gtp_lm_head_logprob_rows that also writes
 * the fp32 logits x = h W^T, vocabulary-major: out_logits[v * logits_stride
 * + n] = x[n, v], for a backward pass.  Under autograd the reference keeps
 * the same bytes: torch.logsumexp saves each chunk's fp32 logits for its
 * backward (tensor_utils.py:180-184, called with grad enabled at
 * models/qwen35_36/training.py:407-427).
 * Arguments as gtp_lm_head_logprob_rows, plus
 *   out_logits    [V, logits_stride] fp32, 4-byte aligned, logits_stride >= N
 *                 (the first N of each vocabulary row are written).
 */
int gtp_lm_head_logprob_save_rows(const uint16_t* hidden, int64_t N, int64_t K,
                                  int64_t hidden_stride, const uint16_t* weight, int64_t V,
                                  int64_t weight_stride, const void* targets,
                                  int targets_int64, float* out_logprob, float* out_entropy,
                                  float* out_lse, int32_t* out_status, float* out_logits,
                                  int64_t logits_stride, void* workspace,
                                  size_t workspace_bytes, void* stream);

/*
 * gtp_logprob_backward_rows -- gradient of log_softmax(x)[target] with respect
 * to the logits, scaled by the incoming gradient of each row:
 *   grad[i] = g * ([i == target - col_offset] - exp(x_i - lse))
 * written in the logits' dtype (bf16 rounded to nearest even), one read of
 * the logits and one write of the gradient.
 *
 * Replaces the autograd backward of sequence_log_probs_from_logits
 * src/graspo/core/graspo_loss.py:19-21 and of F.cross_entropy in
 * sft_cross_entropy_loss src/graspo/core/sft_loss.py:12-34 (both materialise
 * the [N, V] softmax in fp32), and the per-chunk softmax of the backward of
 * _selected_token_log_probs_from_hidden tensor_utils.py:167-186 (logits of one
 * vocabulary chunk, col_offset = its first column).
 *
 *   targets       [N] int32 (targets_int64 == 0) or int64; a target outside
 *                 [col_offset, col_offset + V) adds no one-hot term
 *   grad_logprob  [N] fp32, g per row; a row with g == 0 is written as zeros
 *                 without reading its logits (ignored positions)
 *   lse           [N] fp32, the row's log-sum-exp over the whole vocabulary
 *   grad          [N, grad_stride] of dtype, 16-byte aligned rows take the
 *                 vector path
 */
int gtp_logprob_backward_rows(const void* logits, int dtype, int64_t N,
                              int64_t V, int64_t row_stride,
                              int64_t col_offset, const void* targets,
                              int targets_int64, const float* grad_logprob,
                              const float* lse, void* grad,
                              int64_t grad_stride, void* stream);

/*
 * gtp_softmax_grad_bf16_cols -- grad_t[v, n] = bf16(-g_n exp(x_t[v, n] - lse_n))
 * of vocabulary-major fp32 logits (the layout gtp_lm_head_logprob_save_rows
 * writes), rounded to nearest even: the softmax part of the gradient of
 * g_n log_softmax(x_n)[t_n] without its one-hot term g_n [v == t_n], which
 * the caller adds in fp32.  Each element is within 2^-8 of -g p.  Feeds the
 * hidden-state path's backward (tensor_utils.py:167-186 under autograd):
 * bf16 matrix-core GEMMs of it against the exact bf16 operands, fp32 output.
 * With grad_n the same values are also written token-major, from the same
 * read of the logits (the two gradient GEMMs each run fastest on one of the
 * two layouts).
 *   logits_t  [V, logits_stride] fp32 (the first N of each row are read)
 *   grad_logprob, lse  [N] fp32; a token with g == 0 gets zeros
 *   grad_t    [V, grad_stride] bf16, or NULL (then grad_n is required)
 *   grad_n    [N, grad_n_stride] bf16, or NULL
 */
int gtp_softmax_grad_bf16_cols(const float* logits_t, int64_t V, int64_t N,
                               int64_t logits_stride, const float* grad_logprob,
                               const float* lse, uint16_t* grad_t, int64_t grad_stride,
                               uint16_t* grad_n, int64_t grad_n_stride, void* stream);

/*
 * gtp_logprob_backward_split_rows -- the gradient of gtp_logprob_backward_rows
 * for fp32 logits, written as two bf16 arrays: grad_hi = the gradient rounded
 * to bf16, grad_lo = the remainder rounded to bf16, so that
 * |grad - hi - lo| <= 2^-16 |grad| (lo = 0 where hi is not finite): about 16
 * significant bits.  Feeds the hidden-state path's backward
 * (tensor_utils.py:167-186 under autograd) into bf16 matrix-core GEMMs with
 * fp32 output.
 * Arguments as gtp_logprob_backward_rows; grad_hi and grad_lo share
 * grad_stride.
 */
int gtp_logprob_backward_split_rows(const float* logits, int64_t N, int64_t V,
                                    int64_t row_stride, int64_t col_offset,
                                    const void* targets, int targets_int64,
                                    const float* grad_logprob, const float* lse,
                                    uint16_t* grad_hi, uint16_t* grad_lo,
                                    int64_t grad_stride, void* stream);

/*
 * gtp_graspo_loss_forward / gtp_graspo_loss_backward -- the GRASPO PPO-clip
 * surrogate over token logprobs, fused:
 *   loss = mean_b( sum_t m l / max(1, sum_t m) ),
 *   l = -min(r A, clamp(r, clip_lo, clip_hi) A),  r = exp(logp - old_logp)
 * Replaces GRASPOLoss.forward src/graspo/core/graspo_loss.py:45-63 with
 * masked_mean :10-16 (about ten elementwise and reduction launches) by two
 * kernels forward and one backward.
 *
 *   logp, old_logp, adv  [B, T] fp32 contiguous
 *   mask                 [B, T] fp32 weights (mask_u8 == 0), bytes of 0/1
 *                        (mask_u8 != 0, e.g. a bool tensor), or NULL (all ones)
 *   clip_lo, clip_hi     1 - eps and 1 + eps as fp32
 *   out_loss             [1] fp32; per_seq [B] fp32 (each sequence's masked
 *                        mean); inv_denom [B] fp32 (1 / max(1, sum_t m)),
 *                        which the backward reads
 *   grad_loss            [1] fp32, d(out)/d(loss) from the caller
 *   grad_logp            [B, T] fp32: d(out)/d(logp); old_logp, adv and the
 *                        mask get no gradient (as in the reference's use)
 */
int gtp_graspo_loss_forward(const float* logp, const float* old_logp,
                            const float* adv, const void* mask, int mask_u8, int64_t B,
                            int64_t T, float clip_lo, float clip_hi,
                            float* out_loss, float* per_seq, float* inv_denom,
                            void* stream);
int gtp_graspo_loss_backward(const float* logp, const float* old_logp,
                             const float* adv, const void* mask, int mask_u8,
                             const float* inv_denom, const float* grad_loss,
                             int64_t B, int64_t T, float clip_lo,
                             float clip_hi, float* grad_logp, void* stream);

/*
 * gtp_decode_update_rows -- the generation loop's per-token bookkeeping after
 * gtp_sample_rows, in one launch and without a host synchronisation.
 *
 * Replaces the statements that follow the sampler in the decode loops
 *   src/graspo/backends/graspoflow/models/qwen3/adapter.py:293-304, :338-351
 *   src/graspo/backends/graspoflow/models/qwen35_36/generation.py:259-270,
 *   :304-317, :558-569, :606-630
 * (sequences = cat([sequences, next_token]); finished |= next_token == eos;
 * all_finished = bool(finished.all()); attention_mask = sequences.ne(pad)).
 *
 *   ids       [B] int64 in/out, the sampler's out_ids (rows finished before
 *             the step already hold pad_token_id).  A row whose status is
 *             not GTP_ROW_OK (its id is -1) gets pad_token_id here, in ids,
 *             seq and attn alike, so no id outside [0, V) reaches the next
 *             forward before the caller reads flags[1] and raises.
 *   status    [B] int32, the sampler's out_status, or NULL
 *   finished  [B] uint8 (or bool) in/out: finished[b] |= ids[b] == eos_token_id
 *   seq       [B, seq_stride] int64 or NULL: seq[b, col] = ids[b]
 *   attn      [B, attn_stride] uint8 (or bool) or NULL:
 *             attn[b, col] = ids[b] != pad_token_id
 *   flags     [2] int32 out: rows not finished after the update, and rows
 *             whose status is not GTP_ROW_OK.  The caller copies them to
 *             host memory asynchronously; flags[0] == 0 is the reference's
 *             all_finished.
 */
int gtp_decode_update_rows(int64_t* ids, const int32_t* status, int64_t B,
                           int64_t eos_token_id, int64_t pad_token_id,
                           uint8_t* finished, int64_t* seq, int64_t seq_stride,
                           uint8_t* attn, int64_t attn_stride, int64_t col,
                           int32_t* flags, void* stream);

/*
 * gtp_f32_to_bf16_exact -- dst[i] = the upper 16 bits of src[i] (the bf16
 * value of an fp32 value that is one), for n elements; *inexact |= 1 when any
 * src[i] has nonzero lower 16 bits (it is not a bf16 value, and dst[i] is
 * then not its rounding).  The caller zeroes *inexact.  One HBM pass.
 *
 * Serves the hidden-state logprob path: the reference hands
 * _selected_token_log_probs_from_hidden (tensor_utils.py:167-186) fp32 copies
 * of bf16 tensors (qwen3/model.py:361-365, qwen35_36/training.py:619-623) and
 * multiplies them in fp32; when both operands are bf16 values the chunk GEMMs
 * run on bf16 matrix cores with fp32 output instead, with the same products.
 */
int gtp_f32_to_bf16_exact(const float* src, int64_t n, uint16_t* dst,
                          uint32_t* inexact, void* stream);

/*
 * gtp_time_next_launch -- measurement hook, no counterpart in the reference:
 * the next gtp_sample_rows, gtp_logprob_entropy_rows, gtp_logprob_backward_rows
 * or gtp_stream_read_rows call from the calling thread records start_event
 * when its kernel's dispatch begins and stop_event when it ends
 * (hipExtLaunchKernelGGL; each of these calls is one launch), so the two HIP
 * events bracket the call's kernel, without the idle time of event packets
 * recorded around it.
 * Both are hipEvent_t created by the caller (with timing).  The hook is per
 * thread and used once; the benchmark is its caller.
 */
int gtp_time_next_launch(void* start_event, void* stop_event);

/*
 * gtp_stream_read_rows -- measurement helper, no counterpart in the
 * reference: reads `rows` rows of `row_bytes` bytes (row_stride_bytes
 * apart, all multiples of 16 from a 16-byte aligned `data`) once, with the
 * samplers' access pattern (one 1024-thread workgroup per row, 16-byte
 * non-temporal loads), and computes nothing else: the streaming floor the
 * sampler kernels are measured against.  `out` ([rows] uint32) is written
 * only for a row whose XOR of words equals 0x9E3779B9.  Goes through the
 * gtp_time_next_launch hook.
 */
int gtp_stream_read_rows(const void* data, int64_t rows, int64_t row_bytes,
                         int64_t row_stride_bytes, uint32_t* out, void* stream);

/* Library version string, e.g. "graspo_tokpath 0.1 gfx950". */
const char* gtp_version(void);

#ifdef __cplusplus
}
#endif

#endif /* GRASPO_TOKPATH_H */
