/*
 * roserlhf_amd.h — C ABI of the gfx950 (MI355X) kernels behind the
 * rosellm_amd.roserlhf Python package.
 *
 * The reference (rosellm.roserlhf) is pure PyTorch and has no native layer; each
 * entry point below replaces the ATen op sequence of one reference function,
 * cited as file:line into rosellm/roserlhf/.  Python (rosellm_amd/_native.py)
 * binds these with ctypes.
 *
 * Conventions shared by every entry point:
 *   - Every pointer is a device pointer unless named *_host.  All outputs and
 *     workspaces are allocated by the caller; nothing here allocates.
 *   - Calls are asynchronous and ordered on `stream` (a hipStream_t; NULL is the
 *     legacy default stream).  They are reentrant and thread-safe.
 *   - Return 0 on success or a negative rrl_status; rrl_last_error() then holds
 *     a message for the calling thread.
 *   - Data-dependent errors (an empty mask, a target id outside [0, V), an
 *     invalid turn id) cannot be seen on the host without a sync, so kernels OR
 *     rrl_flag bits into a caller-provided device int32 `status` word.  The
 *     caller reads it once after the call and raises.
 *   - A 2-D operand [rows, cols] is passed as an rrl_view: element (r, c) lives
 *     at ptr + r*s_row + c*s_col elements.  s_col = 0 broadcasts a per-row value
 *     over columns and s_row = 0 broadcasts one row (torch expand() views).
 *   - Arithmetic is float32 unless an input is float64, in which case it is
 *     float64 ("acc" type below).  16-bit inputs are widened on load.
 */
#ifndef ROSERLHF_AMD_H
#define ROSERLHF_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RRL_ABI_VERSION 4

#if defined(__GNUC__)
#define RRL_API __attribute__((visibility("default")))
#else
#define RRL_API
#endif

/* Element types.  BOOL is one byte, nonzero = true. */
enum rrl_dtype {
  RRL_F32 = 0,
  RRL_F64 = 1,
  RRL_BF16 = 2,
  RRL_F16 = 3,
  RRL_BOOL = 4,
  RRL_U8 = 5,
  RRL_I8 = 6,
  RRL_I16 = 7,
  RRL_I32 = 8,
  RRL_I64 = 9
};

enum rrl_status {
  RRL_OK = 0,
  RRL_EINVAL = -1,  /* bad size, stride, null pointer or parameter */
  RRL_EDTYPE = -2,  /* dtype not supported for this operand */
  RRL_ELAUNCH = -3, /* kernel launch failed (HIP error text in rrl_last_error) */
  RRL_EALIGN = -4   /* pointer alignment below the element size */
};

/* Bits written (OR-ed) into the device `status` word. */
enum rrl_flag {
  RRL_FLAG_EMPTY_MASK = 1,       /* global mask weight sum is zero        (losses.py:48-49)   */
  RRL_FLAG_EMPTY_ROW = 2,        /* some row has no action token          (losses.py:250-251) */
  RRL_FLAG_TARGET_RANGE = 4,     /* target id outside [0, V)              (gather, losses.py:36) */
  RRL_FLAG_INVALID_TURN = 8,     /* unmasked token with invalid turn id   (advantages.py:284-286) */
  RRL_FLAG_FAST_RANGE = 16,      /* rrl_fused_logprob_policy's 16-bit register-resident kernel met a
                                    row with finite |log-sum-exp| > 2e38, outside its exponent range;
                                    that call's outputs are undefined: rerun it with
                                    RRL_POLICY_GENERIC set, or queue a rerun with
                                    RRL_POLICY_RERUN_FAST_RANGE (no reference counterpart) */
  RRL_FLAG_BAD_PROBS = 32,       /* rrl_sample_logprobs: a row holds NaN or +inf logits (torch.multinomial
                                    rejects such probabilities, roseinfer/engine.py:1155,1169) */
  RRL_FLAG_LM_RANGE = 64         /* rrl_lm_head_fwd without mref_in: a token's logits rose more than 64
                                    above its first 32-column tile maximum + 24, outside the fixed
                                    reference point's exponent range; that token's outputs are
                                    undefined: rerun with mref_in = the log-sum-exp of an LSE-only
                                    call (no reference counterpart) */
};

/* rrl_policy_params.flags bits. */
enum rrl_policy_flag {
  RRL_POLICY_GENERIC = 1,     /* rrl_fused_logprob_policy: use the generic row kernel only */
  RRL_POLICY_SKIP_MASKED = 2, /* rrl_fused_logprob_policy: a token whose mask weight is exactly 0
                                 is not read; its dlogits row is written as zeros and its logp /
                                 lse as 0 (equal to the reference for finite logits, where such a
                                 row contributes exactly 0; no reference counterpart) */
  RRL_POLICY_SUM = 4,         /* RRL_OBJ_NLL: reduction "sum" instead of "mean" */
  RRL_POLICY_RERUN_FAST_RANGE = 8 /* rrl_fused_logprob_policy: launch the generic row kernel as a
                                 conditional rerun of the call just made with the same arguments
                                 on the same stream and status word (status required): its
                                 workgroups return at once unless the status word holds
                                 RRL_FLAG_FAST_RANGE, so a caller need not read the status between
                                 the two launches (no reference counterpart) */
};

/* Policy objectives (losses.py). */
enum rrl_objective {
  RRL_OBJ_PPO = 0,        /* clipped_policy_loss      losses.py:426-486 */
  RRL_OBJ_SAO = 1,        /* sao_policy_loss          losses.py:127-203 */
  RRL_OBJ_GSPO = 2,       /* gspo_policy_loss         losses.py:206-273 */
  RRL_OBJ_GSPO_TOKEN = 3, /* gspo_token_policy_loss   losses.py:276-352 */
  RRL_OBJ_SAPO = 4,       /* sapo_policy_loss         losses.py:355-423 */
  RRL_OBJ_NLL = 5         /* SFT next-token cross-entropy: F.cross_entropy(logits, labels) with
                             ignore_index and reduction "mean" (or "sum"), as called by
                             rosetrainer/model.py:643-649 and rosetrainer/qwen3.py:558-564.
                             The objective is sum(w * logp) / sum(w) (or sum(w * logp)), the loss
                             its negative.  The `mask` operand is the target ids themselves (I32
                             or I64): w = 1 where the id differs from ignore_index, else 0, and an
                             ignored id is not range-checked.  An all-ignored batch gives a NaN
                             "mean" objective and zero gradients, as F.cross_entropy does; no
                             EMPTY_MASK flag is raised. */
};

/* Scalar outputs of rrl_policy_fwd, in this order (acc dtype):
 *   PPO:        objective, approximate_kl, clip_fraction, mean_ratio
 *   SAO:        objective, approximate_kl, rejected_fraction, mean_ratio
 *   GSPO(/tok): objective, sequence_ratio_divergence, sequence_clip_fraction,
 *               mean_sequence_ratio
 *   SAPO:       objective, approximate_kl, mean_ratio, mean_gradient_gate
 *   NLL:        objective, number of non-ignored tokens
 * Slots 4..7 are reserved.  rrl_policy_bwd takes upstream gradients in the
 * same slots (non-differentiable slots are ignored). */
#define RRL_NSCALARS 8

typedef struct rrl_view {
  const void* ptr;
  int32_t dtype;
  int64_t s_row;
  int64_t s_col;
} rrl_view;

typedef struct rrl_policy_params {
  int32_t kind;          /* rrl_objective */
  int32_t detach_ratio;  /* SAO only (losses.py:185) */
  int32_t mask_is_weight;/* 1: mask is cast to the value dtype and used as a
                            weight (masked_mean, losses.py:46); 0: mask != 0 */
  int32_t flags;         /* rrl_policy_flag bits */
  double clip_low;       /* thresholds are formed as acc(1 - clip_low) etc. */
  double clip_high;
  double max_log_ratio;
  double tau_positive;   /* SAPO */
  double tau_negative;   /* SAPO */
  int64_t ignore_index;  /* NLL: target id that carries no loss (F.cross_entropy's ignore_index) */
} rrl_policy_params;

RRL_API const char* rrl_last_error(void);
RRL_API int rrl_abi_version(void);

/* ---- a1/a2: token log-probs (losses.py:14-38) and their backward ---------
 * logits: [B, T, V] with the vocabulary contiguous; row (b, t) starts at
 * logits + b*ls_b + t*ls_t elements (a causal shift logits[:, :-1] is such a
 * view).  dtype F32, F64, BF16 or F16.  targets: [B, T] view, I32 or I64.
 * Outputs are contiguous [B*T]: logp in logp_dtype (F32 or F64), lse in acc. */
RRL_API int rrl_logprob_fwd(const void* logits, int32_t logits_dtype, int64_t B, int64_t T,
                    int64_t V, int64_t ls_b, int64_t ls_t, rrl_view targets,
                    void* logp_out, int32_t logp_dtype, void* lse_out,
                    int32_t* status, void* stream);

/* rrl_logprob_fwd over the rows whose mask is nonzero: a row whose mask
 * element (B x T view, any dtype; -0.0 counts as 0) is exactly 0 is not read
 * and its logp and lse are written as 0.  For objectives in which such a
 * token's log-prob enters only multiplied by its zero mask weight (GSPO's
 * sequence log-ratio, losses.py:249-256, and its token form), the results are
 * those of rrl_logprob_fwd for finite logits.  No reference counterpart. */
RRL_API int rrl_logprob_fwd_masked(const void* logits, int32_t logits_dtype, int64_t B,
                    int64_t T, int64_t V, int64_t ls_b, int64_t ls_t, rrl_view targets,
                    rrl_view mask, void* logp_out, int32_t logp_dtype, void* lse_out,
                    int32_t* status, void* stream);

/* dlogits[b,t,v] (+)= g[b*T+t] * ([v == target] - exp(x[b,t,v] - lse[b*T+t])),
 * the composed gather_backward + log_softmax_backward (autograd of
 * losses.py:34-38).  g, lse and logp are contiguous acc-typed [B*T] (logp as
 * written by rrl_logprob_fwd; may be NULL, in which case the target column is
 * formed from lse, losing relative precision when p_target -> 1); dlogits has
 * its own (ds_b, ds_t) row strides and dtype.  accumulate = 1 adds into
 * dlogits.  dlogits may alias logits when the strides match (in-place). */
RRL_API int rrl_logprob_bwd(const void* logits, int32_t logits_dtype, int64_t B, int64_t T,
                    int64_t V, int64_t ls_b, int64_t ls_t, rrl_view targets,
                    const void* lse, const void* logp, const void* g, void* dlogits,
                    int32_t dl_dtype, int64_t ds_b, int64_t ds_t, int32_t accumulate,
                    void* stream);

/* dlogits[b,t,:] *= scale[0] unless scale[0] == skip_if (no memory touched
 * then).  scale is a device acc scalar, so the caller never syncs. */
RRL_API int rrl_scale_rows(void* dlogits, int32_t dl_dtype, int64_t B, int64_t T, int64_t V,
                   int64_t ds_b, int64_t ds_t, const void* scale, int32_t scale_dtype,
                   double skip_if, void* stream);

/* ---- a3-a8: policy objectives over [B, T] log-probs ---------------------
 * cur, old: [B, T] log-prob views; adv: [B, T] view, or [B] broadcast with
 * s_col = 0 for GSPO (sequence advantages); mask: [B, T] any dtype.
 * workspace: rrl_policy_workspace_bytes(B, acc) bytes, written by fwd and read
 * by bwd (per-row statistics).  scalars_out: acc[RRL_NSCALARS].
 * seq_out: acc[B] sequence ratios for GSPO kinds (else may be NULL).
 * trusted_out: uint8 [B*T] SAO trust mask intersected with the action mask
 * (else may be NULL).  status gets EMPTY_MASK / EMPTY_ROW. */
RRL_API size_t rrl_policy_workspace_bytes(int64_t B, int32_t acc_dtype);

RRL_API int rrl_policy_fwd(const rrl_policy_params* params, int64_t B, int64_t T, rrl_view cur,
                   rrl_view old, rrl_view adv, rrl_view mask, int32_t acc_dtype,
                   void* workspace, void* scalars_out, void* seq_out,
                   uint8_t* trusted_out, int32_t* status, void* stream);

/* grad_cur[b*T+t] (acc, contiguous) = sum_k grad_scalars[k] * d scalar_k / d cur[b,t]
 * (+ sum_b grad_seq[b] * d seq_ratio_b / d cur for GSPO kinds; grad_seq may be
 * NULL).  grad_scalars: device acc[RRL_NSCALARS]. */
RRL_API int rrl_policy_bwd(const rrl_policy_params* params, int64_t B, int64_t T, rrl_view cur,
                   rrl_view old, rrl_view adv, rrl_view mask, int32_t acc_dtype,
                   const void* workspace, const void* grad_scalars, const void* grad_seq,
                   void* grad_cur, void* stream);

/* ---- single pass: log-prob + token-local objective gradient --------------
 * For PPO, SAO, SAPO and NLL, d loss / d logp is token-local once the mask
 * denominators are known, so one sweep over each logits row produces logp,
 * lse and dlogits = d(-objective)/d logits.  rrl_policy_row_coef first writes
 * row_coef[b] (acc, [B]): 1/sum(mask weight) for PPO/SAO/NLL (1 for NLL with
 * RRL_POLICY_SUM), 1/(B*L_b) for SAPO, and flags EMPTY_MASK / EMPTY_ROW.  The objective scalars then come from
 * rrl_policy_fwd on the returned logp.
 * records: caller workspace of rrl_fused_records_bytes(B, T) bytes, where the
 * register-resident path (16-bit and float32 logits, V <= 163840 16-bit or
 * 81920 float32 entries) packs each token's target, old log-prob, advantage
 * and mask weight * row_coef (16 bytes per token) for one scalar load per
 * row. */
RRL_API int rrl_policy_row_coef(const rrl_policy_params* params, int64_t B, int64_t T,
                        rrl_view mask, int32_t acc_dtype, void* row_coef,
                        void* workspace, int32_t* status, void* stream);

RRL_API size_t rrl_fused_records_bytes(int64_t B, int64_t T);

/* Target ids checked ahead of the single-pass sweep: TARGET_RANGE in *status
 * for any target[b, t] (int32 or int64 view) outside [0, V) that is not NLL's
 * ignore_index (params->ignore_index for kind RRL_OBJ_NLL).  The sweep makes
 * the same check; this entry lets a caller read the status before launching
 * it, so the host need not wait for the sweep to raise the index error of
 * torch.gather (losses.py:34-38) or F.cross_entropy (model.py:643-649).  It
 * replaces no reference function of its own. */
RRL_API int rrl_check_targets(const rrl_policy_params* params, int64_t B, int64_t T, int64_t V,
                      rrl_view target, int32_t* status, void* stream);

RRL_API int rrl_fused_logprob_policy(const rrl_policy_params* params, const void* logits,
                             int32_t logits_dtype, int64_t B, int64_t T, int64_t V,
                             int64_t ls_b, int64_t ls_t, rrl_view targets, rrl_view old,
                             rrl_view adv, rrl_view mask, const void* row_coef,
                             void* records, void* logp_out, void* lse_out, void* dlogits,
                             int32_t dl_dtype, int64_t ds_b, int64_t ds_t,
                             int32_t* status, void* stream);

/* rrl_fused_logprob_policy without the records workspace: no counterpart in
 * the reference.  It is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The per-token records live in a static device array of
 * RRL_NOALLOC_MAX_TOKENS x 16 bytes (16 MiB), one copy per GPU, held until the
 * process ends; B*T above RRL_NOALLOC_MAX_TOKENS returns RRL_EINVAL.  Every
 * call on one GPU shares that array: calls that overlap on one GPU (two
 * streams, two threads) race and must be serialised by the caller.  Arguments
 * and results are those of rrl_fused_logprob_policy; nothing is allocated. */
#define RRL_NOALLOC_MAX_TOKENS (1 << 20)
RRL_API int rrl_fused_logprob_policy_noalloc(const rrl_policy_params* params,
                             const void* logits, int32_t logits_dtype, int64_t B, int64_t T,
                             int64_t V, int64_t ls_b, int64_t ls_t, rrl_view targets,
                             rrl_view old, rrl_view adv, rrl_view mask, const void* row_coef,
                             void* logp_out, void* lse_out, void* dlogits, int32_t dl_dtype,
                             int64_t ds_b, int64_t ds_t, int32_t* status, void* stream);

/* ---- a4, a9: masked_mean (losses.py:41-50), sequence_log_ratio (:489-512)
 * masked_mean: out = acc[1] = sum(values * w) / sum(w), w = mask cast to the
 * value dtype; flags EMPTY_MASK.  The workspace keeps the denominator for the
 * backward.  sequence_log_ratio: out, counts_out = acc[B]; flags EMPTY_ROW. */
RRL_API size_t rrl_reduce_workspace_bytes(int64_t n);
RRL_API int rrl_masked_mean_fwd(int64_t B, int64_t T, rrl_view values, rrl_view mask,
                        int32_t acc_dtype, void* workspace, void* out, int32_t* status,
                        void* stream);
/* grad_values[b*T+t] = grad[0] * w[b,t] / sum(w); workspace as written by fwd. */
RRL_API int rrl_masked_mean_bwd(int64_t B, int64_t T, rrl_view mask, int32_t acc_dtype,
                        const void* workspace, const void* grad, void* grad_values,
                        void* stream);
RRL_API int rrl_sequence_log_ratio_fwd(int64_t B, int64_t T, rrl_view cur, rrl_view old,
                               rrl_view mask, int32_t length_normalize, int32_t acc_dtype,
                               void* out, void* counts_out, int32_t* status, void* stream);
RRL_API int rrl_sequence_log_ratio_bwd(int64_t B, int64_t T, rrl_view mask, int32_t length_normalize,
                               int32_t acc_dtype, const void* counts, const void* grad,
                               void* grad_cur, void* stream);

/* direct_double_sided_mask (losses.py:104-124): out = (r > lo) & (r < hi), strict.
 * lo = 1 - clip_low and hi = 1 + clip_high must already be rounded to the
 * ratio dtype (torch compares a tensor with a Python scalar in the tensor's
 * dtype). */
RRL_API int rrl_double_sided_mask(int64_t n, const void* ratios, int32_t dtype, double lo, double hi,
                          uint8_t* out, void* stream);

/* ---- a10-a17: estimators (advantages.py) ----------------------------------
 * Sequences are rows of [B, T] views; reverse recurrences run as segmented
 * affine scans.  terminated / valid may have ptr = NULL (all false / all true).
 * bootstrap: [B] view (s_col ignored) or ptr = NULL for zero.  Outputs are
 * contiguous [B*T] in out_dtype. */
RRL_API int rrl_discounted_returns(int64_t B, int64_t T, rrl_view rewards, rrl_view terminated,
                           rrl_view valid, rrl_view bootstrap, double gamma,
                           void* out, int32_t out_dtype, void* stream);

RRL_API int rrl_gae(int64_t B, int64_t T, rrl_view rewards, rrl_view values, rrl_view terminated,
            rrl_view valid, rrl_view bootstrap, double gamma, double gae_lambda,
            void* adv_out, void* targets_out, int32_t out_dtype, void* stream);

RRL_API int rrl_skip_observation_gae(int64_t B, int64_t T, rrl_view rewards,
                             rrl_view action_end_values, rrl_view next_action_values,
                             rrl_view terminated, rrl_view valid, double gamma,
                             double gae_lambda, void* adv_out, void* targets_out,
                             int32_t out_dtype, void* stream);

/* Groups are rows of a [n_groups, G] view. */
RRL_API int rrl_group_standardize(int64_t n_groups, int64_t G, rrl_view rewards, double eps,
                          void* out, int32_t out_dtype, void* stream);
RRL_API int rrl_leave_one_out(int64_t n_groups, int64_t G, rrl_view rewards, void* out,
                      int32_t out_dtype, void* stream);

/* out[b,t] = mask[b,t] ? turn_adv[b, turn_ids[b,t]] : 0; flags INVALID_TURN. */
RRL_API int rrl_broadcast_turn(int64_t B, int64_t K, int64_t T, rrl_view turn_adv,
                       rrl_view turn_ids, rrl_view mask, void* out, int32_t out_dtype,
                       int32_t* status, void* stream);

/* Masked whitening over all tokens with mask != 0 (no reference function):
 * out = mask ? (x - mean) / (std_pop + eps) : 0, mean and population std over
 * the masked tokens; shift_mean = 0 keeps the mean (out = mask ? x/(std+eps)
 * : 0).  workspace: rrl_reduce_workspace_bytes(B*T).  Flags EMPTY_MASK. */
RRL_API int rrl_masked_whiten(int64_t B, int64_t T, rrl_view x, rrl_view mask, double eps,
                      int32_t shift_mean, int32_t acc_dtype, void* workspace, void* out,
                      int32_t out_dtype, int32_t* status, void* stream);

/* ---- fused LM head + token log-probs (rosetrainer/model.py:641,
 * rosetrainer/qwen3.py:556 feeding losses.py:14-38), on the matrix cores ----
 * The reference forms logits = hidden @ weight^T as a [N, V] tensor, then
 * log_softmax + gather, and autograd's backward forms the [N, V] dlogits and
 * the two products dlogits @ weight, dlogits^T @ hidden.  These entry points
 * never hold more than a 32 x 64 logits tile (registers and LDS):
 *   hidden: [N, H] rows h_ld elements apart; weight: [V, H] rows w_ld apart;
 *   both BF16 (dtype RRL_BF16), 16-byte aligned, H a multiple of 128 up to 1024,
 *   row strides multiples of 8 elements.  targets: contiguous int32 [N]
 *   (a negative id: no target, logp 0 and no gradient, as cross-entropy's
 *   ignore_index; the caller range-checks ids with rrl_check_targets).
 * rrl_lm_head_fwd writes lse_out and logp_out (float32 [N]) and, when obar is
 * not NULL, obar[n] = sum_{v != target} p_nv weight[v] (float32 [N, H], row
 * stride obar_ld): the softmax-weighted weight rows the backward's dhidden
 * needs, from the same pass (flash-attention-style online softmax).  Without
 * obar only the log-sum-exp is formed (half the MFMA work).  A target id >= V
 * raises TARGET_RANGE; a token whose logits exceed the fixed reference point's
 * range raises LM_RANGE (rerun with mref_in = the lse of an obar-less call).
 * mref_in: NULL, or float32 [N] reference points (the rerun).  need_obar:
 * NULL, or uint8 [N]: 1 = the token's obar is needed, 0 = its lse and logp
 * only, 2 = neither.  A block of 64 consecutive tokens none of which needs
 * obar takes the log-sum-exp-only pass and its obar rows are left unwritten
 * (for tokens whose d loss / d logp is zero by construction, such as masked
 * tokens); a block whose 64 tokens are all 2 is not computed at all, and its
 * tokens get lse = logp = 0 (a masked token's log-prob that the caller
 * discards; no reference counterpart).  workspace: with need_obar
 * and obar, rrl_lm_head_fwd_workspace_bytes(N) bytes of caller device memory
 * (16-byte aligned; the order in which the blocks are taken), else ignored. */
RRL_API size_t rrl_lm_head_fwd_workspace_bytes(int64_t N);
RRL_API int rrl_lm_head_fwd(const void* hidden, const void* weight, int32_t dtype, int64_t N,
                    int64_t H, int64_t V, int64_t h_ld, int64_t w_ld, const int32_t* targets,
                    const uint8_t* need_obar, const float* mref_in, float* lse_out,
                    float* logp_out, float* obar, int64_t obar_ld, void* workspace,
                    int32_t* status, void* stream);

/* dhidden[n] = g[n] * ((-expm1(logp[n])) * weight[target[n]] - obar[n]), in the
 * weight dtype, rows dh_ld apart (the linear map's backward of a1's gradient
 * g = d loss / d logp, with the target column's 1 - p formed from logp). */
RRL_API int rrl_lm_head_dhidden(const void* weight, int32_t dtype, int64_t N, int64_t H,
                    int64_t V, int64_t w_ld, const int32_t* targets, const float* logp,
                    const float* g, const float* obar, int64_t obar_ld, void* dhidden,
                    int64_t dh_ld, void* stream);

/* dweight[v] = sum_n g[n] ([v == target[n]] - exp(logit[n, v] - lse[n])) hidden[n],
 * the logits recomputed tile by tile, float32 accumulation over every token in
 * registers, written once as float32 or the weight dtype (dw_dtype), rows dw_ld
 * apart.  Tiles of 32 consecutive tokens whose g are all zero contribute
 * exactly zero and are not visited.  workspace:
 * rrl_lm_head_dweight_workspace_bytes(N, H, V) bytes of caller device memory
 * (16-byte aligned; token records, the visited tiles, and float32 partial rows
 * of the weight blocks that a last partial round of workgroups splits over
 * token ranges; the size depends on the current device's CU count). */
RRL_API size_t rrl_lm_head_dweight_workspace_bytes(int64_t N, int64_t H, int64_t V);
RRL_API int rrl_lm_head_dweight(const void* hidden, const void* weight, int32_t dtype,
                    int64_t N, int64_t H, int64_t V, int64_t h_ld, int64_t w_ld,
                    const int32_t* targets, const float* lse, const float* logp,
                    const float* g, void* workspace, void* dweight, int32_t dw_dtype,
                    int64_t dw_ld, void* stream);

/* ---- operand layout for the chunked LM head's library GEMMs ----
 * No counterpart in the reference: the chunked path of the LM head
 * (roserlhf/linear.py, standing in for rosetrainer/model.py:641's F.linear
 * and its backward) hands the GEMM library the weight as a contiguous [H, V]
 * copy for d hidden = dL W, the layout it runs fastest.
 * rrl_transpose16: dst[c * dst_ld + r] = src[r * src_ld + c] for r < rows,
 * c < cols, 2-byte elements (bf16/f16 bits copied unchanged), asynchronous on
 * `stream`.  16-byte accesses when both bases are 16-byte aligned and both
 * strides are multiples of 8 elements. */
RRL_API int rrl_transpose16(const void* src, int64_t rows, int64_t cols, int64_t src_ld,
                    void* dst, int64_t dst_ld, void* stream);

/* ---- rollout side: next-token sampling with behaviour log-probs -------------
 * Replaces the token choice of roseinfer/engine.py:1103-1171
 * (InferenceEngine._sample_next_token_batch, its PyTorch path) and adds the
 * log-probabilities that rosellm/roserlhf/trajectory.py:15,27-28 requires per
 * sampled token.  logits: [B, V] rows of F32, BF16 or F16, row r at
 * logits + r*row_stride elements.  Per row:
 *   - greedy (do_sample == 0 or temperature <= 0): the lowest index of the
 *     maximum (torch.argmax);
 *   - else x/temperature; candidates = the top_k largest when 0 < top_k < V
 *     (ties at the k-th value kept lowest index first), else the whole row;
 *     p = softmax over the candidates; when 0 < top_p < 1, a candidate is
 *     kept iff its inclusive cumulative p in descending order (ties lowest
 *     index first) is <= top_p, the first always; q = max(p * kept, 1e-9) over
 *     the candidates (the reference's masked_fill + clamp_min(1e-9)), 0
 *     elsewhere; the token is the first index, in vocabulary order, whose
 *     inclusive cumulative q exceeds u * sum(q), with one uniform
 *     u = (r >> 8) * 2^-24 per row from Philox4x32-10 (Salmon et al., SC'11)
 *     of counter {row, row >> 32, offset, offset >> 32} and key {seed, seed >> 32}
 *     (r = its first output word).
 * Outputs (contiguous [B]): token_out (int64); logp_out (float32) the token's
 * log_softmax(x / T) over the whole row, T = 1 when greedy, formed as the
 * training kernels form log-probs; logq_out (float32, may be NULL) log(q/sum q),
 * the log-probability of the sampling distribution (0 when greedy).
 * A row with NaN or +inf logits, no finite maximum, or a maximum whose x/T
 * overflows raises BAD_PROBS in *status (status may be NULL) and gets
 * logp_out = logq_out = NaN; every other row's logp_out is not NaN.  The
 * arithmetic is float32 on the exact upcast of the logits (the reference
 * divides and normalises in the logits dtype). */
RRL_API int rrl_sample_logprobs(const void* logits, int32_t logits_dtype, int64_t B, int64_t V,
                        int64_t row_stride, double temperature, int64_t top_k, double top_p,
                        int32_t do_sample, uint64_t seed, uint64_t offset, int64_t* token_out,
                        float* logp_out, float* logq_out, int32_t* status, void* stream);

/* Philox4x32-10 on the host (the generator rrl_sample_logprobs draws from):
 * ctr[4] is replaced by the 4 output words. */
RRL_API void rrl_philox4x32_10(uint32_t ctr[4], const uint32_t key[2]);

#ifdef __cplusplus
}
#endif

#endif /* ROSERLHF_AMD_H */
