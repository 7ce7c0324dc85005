"""Token-level policy objectives on MI355X (drop-in for ``rosellm/roserlhf/losses.py``).

Every public function keeps the reference's name, signature, validation order
and error text; the arithmetic runs in gfx950 HIP kernels reached through the
C ABI in ``include/roserlhf_amd.h``.  Inputs must be ROCm device tensors: there
is no CPU path, and a missing HIP library raises ImportError.

Deliberate differences from the reference, each for numerical quality:
  * bf16/fp16 logits yield float32 log-probs (the reference returns the logits
    dtype); the kernels accumulate in float32 and the fp32 result rounds to the
    reference's bf16 value.
  * objectives on 16-bit log-prob inputs compute in float32.
  * the backward of every objective is the closed-form derivative evaluated in
    one kernel, not autograd over a chain of elementwise ops.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Optional, Tuple

import torch
from torch import Tensor

from .. import _native as nat
from .. import _config as _cfg

__all__ = [
    "GspoPolicyLossOutput",
    "PolicyLossOutput",
    "SapoPolicyLossOutput",
    "SaoPolicyLossOutput",
    "clipped_policy_loss",
    "direct_double_sided_mask",
    "fused_policy_loss",
    "gather_token_logprobs",
    "gspo_policy_loss",
    "gspo_token_policy_loss",
    "masked_mean",
    "sapo_policy_loss",
    "sao_policy_loss",
    "sequence_log_ratio",
]


# ---------------------------------------------------------------------------
# Output records (field names and order as losses.py:53-101)
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class PolicyLossOutput:
    """Policy loss plus diagnostics computed over action tokens."""

    loss: Tensor
    objective: Tensor
    approximate_kl: Tensor
    clip_fraction: Tensor
    mean_ratio: Tensor


@dataclass(frozen=True)
class SaoPolicyLossOutput:
    """SAO policy loss plus trust-mask diagnostics.

    ``trusted_mask`` is already intersected with ``action_mask``.
    """

    loss: Tensor
    objective: Tensor
    approximate_kl: Tensor
    rejected_fraction: Tensor
    mean_ratio: Tensor
    trusted_mask: Tensor


@dataclass(frozen=True)
class GspoPolicyLossOutput:
    """GSPO loss and sequence-level trust-region diagnostics."""

    loss: Tensor
    objective: Tensor
    sequence_ratio_divergence: Tensor
    sequence_clip_fraction: Tensor
    mean_sequence_ratio: Tensor
    sequence_ratios: Tensor


@dataclass(frozen=True)
class SapoPolicyLossOutput:
    """SAPO loss and smooth-gate diagnostics."""

    loss: Tensor
    objective: Tensor
    approximate_kl: Tensor
    mean_ratio: Tensor
    mean_gradient_gate: Tensor


# ---------------------------------------------------------------------------
# a1/a2: token log-probs
# ---------------------------------------------------------------------------


def _raise_target_range() -> None:
    raise RuntimeError("index out of bounds: every target id must lie in [0, vocabulary)")


class _TokenLogprobs(torch.autograd.Function):
    """log_softmax(logits)[target] per row; backward writes dlogits in one sweep.

    With ``skip_mask`` (same shape as the targets) a row whose mask is exactly
    0 is not read: its log-prob and log-sum-exp are 0 (for objectives that
    weight such a token's log-prob by its zero mask; its d loss / d logp is
    then 0 and the backward writes its dlogits row as zeros unread)."""

    @staticmethod
    def forward(ctx, logits: Tensor, target_ids: Tensor,
                skip_mask: Optional[Tensor] = None) -> Tensor:
        dev = nat.require_device(logits, target_ids)
        x, B, T, V, s_b, s_t = nat.logits_rows(logits)
        tview, tkeep = nat.rows_view(target_ids, B, T)
        acc = nat.acc_dtype(logits.dtype)
        logp = torch.empty(B * T, dtype=acc, device=dev)
        lse = torch.empty(B * T, dtype=acc, device=dev)
        status = nat.new_status(dev)
        if skip_mask is None:
            nat.call(
                "rrl_logprob_fwd", x.data_ptr(), nat.dtype_code(x.dtype), B, T, V, s_b, s_t,
                tview, logp.data_ptr(), nat.dtype_code(acc), lse.data_ptr(), status.data_ptr(),
                nat.stream_ptr(dev),
            )
        else:
            mview, _mkeep = nat.rows_view(skip_mask, B, T)
            nat.call(
                "rrl_logprob_fwd_masked", x.data_ptr(), nat.dtype_code(x.dtype), B, T, V, s_b,
                s_t, tview, mview, logp.data_ptr(), nat.dtype_code(acc), lse.data_ptr(),
                status.data_ptr(), nat.stream_ptr(dev),
            )
        if B * T and nat.read_status(status) & nat.FLAG_TARGET_RANGE:
            _raise_target_range()
        # The backward forms the target column from logp (-g * expm1(logp)); a
        # private copy keeps it independent of in-place edits to the output.
        ctx.save_for_backward(x, tkeep, lse, logp.clone())
        ctx.meta = (B, T, V, s_b, s_t, tuple(logits.shape), logits.dtype)
        ctx.set_materialize_grads(False)
        return logp.view(logits.shape[:-1])

    @staticmethod
    def backward(ctx, grad: Optional[Tensor]):
        if grad is None or not ctx.needs_input_grad[0]:
            return None, None, None
        x, tkeep, lse, logp = ctx.saved_tensors
        B, T, V, s_b, s_t, shape, dtype = ctx.meta
        g = grad.reshape(-1).to(lse.dtype).contiguous()
        dl = torch.empty(shape, dtype=dtype, device=x.device)
        tview, _ = nat.rows_view(tkeep, B, T)
        nat.call(
            "rrl_logprob_bwd", x.data_ptr(), nat.dtype_code(x.dtype), B, T, V, s_b, s_t, tview,
            lse.data_ptr(), logp.data_ptr(), g.data_ptr(), dl.data_ptr(), nat.dtype_code(dtype),
            T * V, V, 0, nat.stream_ptr(x.device),
        )
        return dl, None, None


def gather_token_logprobs(logits: Tensor, target_ids: Tensor) -> Tensor:
    """Return log-probability of each target token (losses.py:14-38).

    Args:
        logits: ``[..., vocabulary]`` unnormalized scores.
        target_ids: Integer tensor matching ``logits.shape[:-1]``.

    For a causal LM pass ``logits[:, :-1]`` and ``input_ids[:, 1:]``; both
    views are consumed in place (no copy of the logits).  The result is float32
    (float64 for float64 logits).
    """

    if logits.ndim < 2:
        raise ValueError("logits must include positions and vocabulary")
    if logits.shape[:-1] != target_ids.shape:
        raise ValueError(
            f"target shape {target_ids.shape} must match logits prefix {logits.shape[:-1]}"
        )
    if target_ids.dtype not in (torch.int32, torch.int64):
        raise TypeError("target_ids must be an integer tensor")
    return _cfg.as_reference_dtype(_TokenLogprobs.apply(logits, target_ids), logits)


# ---------------------------------------------------------------------------
# a4: masked_mean
# ---------------------------------------------------------------------------


class _MaskedMean(torch.autograd.Function):
    @staticmethod
    def forward(ctx, values: Tensor, mask: Tensor) -> Tensor:
        dev = nat.require_device(values, mask)
        B, T = nat.flatten_rows(values.shape)
        vview, vkeep = nat.rows_view(values, B, T)
        mview, mkeep = nat.rows_view(mask, B, T)
        acc = nat.acc_dtype(values.dtype)
        ws = torch.empty(nat.lib().rrl_reduce_workspace_bytes(B * T), dtype=torch.uint8, device=dev)
        out = torch.empty(1, dtype=acc, device=dev)
        status = nat.new_status(dev)
        nat.call("rrl_masked_mean_fwd", B, T, vview, mview, nat.dtype_code(acc), ws.data_ptr(),
                 out.data_ptr(), status.data_ptr(), nat.stream_ptr(dev))
        if nat.read_status(status) & nat.FLAG_EMPTY_MASK:
            raise ValueError("cannot reduce an empty mask")
        ctx.save_for_backward(mkeep, ws)
        ctx.meta = (B, T, acc, tuple(values.shape), values.dtype)
        ctx.set_materialize_grads(False)
        return out.reshape(()).to(values.dtype)

    @staticmethod
    def backward(ctx, grad: Optional[Tensor]):
        if grad is None or not ctx.needs_input_grad[0]:
            return None, None
        mkeep, ws = ctx.saved_tensors
        B, T, acc, shape, dtype = ctx.meta
        mview, _ = nat.rows_view(mkeep, B, T)
        g = grad.reshape(1).to(acc).contiguous()
        gv = torch.empty(B * T, dtype=acc, device=ws.device)
        nat.call("rrl_masked_mean_bwd", B, T, mview, nat.dtype_code(acc), ws.data_ptr(),
                 g.data_ptr(), gv.data_ptr(), nat.stream_ptr(ws.device))
        return gv.view(shape).to(dtype), None


def masked_mean(values: Tensor, mask: Tensor) -> Tensor:
    """Globally average valid entries, rejecting an empty denominator (losses.py:41-50)."""

    if values.shape != mask.shape:
        raise ValueError("values and mask must have the same shape")
    return _MaskedMean.apply(values, _on_device(mask, values))


# ---------------------------------------------------------------------------
# a3, a5-a8: objectives
# ---------------------------------------------------------------------------


def _on_device(t: Tensor, like: Tensor) -> Tensor:
    return t if t.device == like.device else t.to(like.device)


def _params(kind: int, *, clip_low: float = 0.0, clip_high: float = 0.0,
            max_log_ratio: float = 20.0, detach_ratio: bool = True, mask_is_weight: bool = False,
            tau_positive: float = 1.0, tau_negative: float = 1.0) -> nat.RrlPolicyParams:
    return nat.RrlPolicyParams(
        kind, int(bool(detach_ratio)), int(bool(mask_is_weight)), 0, float(clip_low),
        float(clip_high), float(max_log_ratio), float(tau_positive), float(tau_negative),
    )


_PER_ROW = (nat.OBJ_GSPO, nat.OBJ_GSPO_TOKEN, nat.OBJ_SAPO)


def _raise_flags(flags: int, kind: int) -> None:
    if flags & nat.FLAG_TARGET_RANGE:
        if kind == nat.OBJ_NLL:  # F.cross_entropy's error type
            raise IndexError("Target is out of bounds: every label other than ignore_index "
                             "must lie in [0, vocabulary)")
        _raise_target_range()
    if kind == nat.OBJ_NLL:
        return
    if kind in _PER_ROW and flags & nat.FLAG_EMPTY_ROW:
        raise ValueError("every sequence needs at least one action token")
    if kind not in _PER_ROW and flags & nat.FLAG_EMPTY_MASK:
        raise ValueError("cannot reduce an empty mask")


def _check_before_sweep(logits: Tensor, inplace: bool) -> bool:
    """Whether the single-pass call reads its status before the sweep.

    Every data error is known before the sweep runs: the row coefficients
    flag empty masks and rrl_check_targets the targets.  The one host
    synchronisation then waits for those small kernels only, and the host
    runs ahead of the sweep.  A log-sum-exp beyond 2e38, which only
    bfloat16's range allows (float16 stops at 65504), makes the
    register-resident kernel flag FAST_RANGE instead; a conditional generic
    launch queued behind it (_rerun_on_device) redoes the call on the GPU in
    that case.  In place the logits are gone by then, so bfloat16 in place
    reads the status after the sweep and raises.
    """

    return logits.dtype != torch.bfloat16 or not inplace


def _rerun_on_device(logits: Tensor, inplace: bool) -> bool:
    """Whether the single-pass call queues RRL_POLICY_RERUN_FAST_RANGE."""

    return logits.dtype == torch.bfloat16 and not inplace


def _rerun_params(params):
    p = nat.RrlPolicyParams.from_buffer_copy(params)
    p.flags |= nat.POLICY_RERUN_FAST_RANGE
    return p


def _scalar_dtypes(kind: int, cur: Tensor, old: Tensor, adv: Tensor) -> Tuple[torch.dtype, ...]:
    ratio = torch.promote_types(cur.dtype, old.dtype)
    obj = torch.promote_types(ratio, adv.dtype)
    if kind == nat.OBJ_SAPO:
        return obj, ratio, ratio, obj
    return obj, ratio, ratio, ratio


def _views(kind: int, cur: Tensor, old: Tensor, adv: Tensor, mask: Tensor):
    B, T = nat.flatten_rows(cur.shape)
    cv, ck = nat.rows_view(cur, B, T)
    ov, ok = nat.rows_view(old, B, T)
    if kind == nat.OBJ_GSPO:
        av, ak = nat.vector_view(adv)
    else:
        av, ak = nat.rows_view(adv, B, T)
    mv, mk = nat.rows_view(mask, B, T)
    return B, T, (cv, ov, av, mv), (ck, ok, ak, mk)


class _PolicyObjective(torch.autograd.Function):
    """Scalars of one objective; backward is the closed-form d/d current_logprobs."""

    @staticmethod
    def forward(ctx, params: nat.RrlPolicyParams, cur: Tensor, old: Tensor, adv: Tensor,
                mask: Tensor):
        kind = params.kind
        dev = nat.require_device(cur, old, adv, mask)
        B, T, views, keep = _views(kind, cur, old, adv, mask)
        acc = nat.acc_dtype(cur.dtype, old.dtype, adv.dtype)
        ws = torch.empty(nat.lib().rrl_policy_workspace_bytes(B, nat.dtype_code(acc)),
                         dtype=torch.uint8, device=dev)
        scal = torch.empty(nat.NSCALARS, dtype=acc, device=dev)
        seq = torch.empty(B if kind in (nat.OBJ_GSPO, nat.OBJ_GSPO_TOKEN) else 0, dtype=acc,
                          device=dev)
        trusted = torch.empty(B * T if kind == nat.OBJ_SAO else 0, dtype=torch.bool, device=dev)
        status = nat.new_status(dev)
        nat.call(
            "rrl_policy_fwd", ctypes_ref(params), B, T, *views, nat.dtype_code(acc), ws.data_ptr(),
            scal.data_ptr(), nat.ptr(seq) if seq.numel() else None,
            nat.ptr(trusted) if trusted.numel() else None, status.data_ptr(), nat.stream_ptr(dev),
        )
        _raise_flags(nat.read_status(status), kind)
        ctx.save_for_backward(*keep, ws)
        ctx.params = params
        ctx.meta = (B, T, acc, tuple(cur.shape), cur.dtype)
        ctx.set_materialize_grads(False)
        dts = _scalar_dtypes(kind, cur, old, adv)
        outs = [scal[k].to(dts[k], copy=True) for k in range(4)]
        ratio_dt = torch.promote_types(cur.dtype, old.dtype)
        seq_out = seq.to(ratio_dt, copy=True)
        trusted_out = trusted.view(cur.shape) if kind == nat.OBJ_SAO else trusted
        # clip / rejected fractions count tokens and carry no gradient
        if kind in (nat.OBJ_PPO, nat.OBJ_SAO):
            ctx.mark_non_differentiable(outs[2], trusted_out)
        elif kind in (nat.OBJ_GSPO, nat.OBJ_GSPO_TOKEN):
            ctx.mark_non_differentiable(outs[2], trusted_out)
        else:
            ctx.mark_non_differentiable(trusted_out)
        return outs[0], outs[1], outs[2], outs[3], seq_out, trusted_out

    @staticmethod
    def backward(ctx, g0, g1, g2, g3, gseq, _gtrusted):
        if not ctx.needs_input_grad[1]:
            return None, None, None, None, None
        ck, ok, ak, mk, ws = ctx.saved_tensors
        B, T, acc, shape, dtype = ctx.meta
        params = ctx.params
        kind = params.kind
        dev = ws.device
        gs = torch.zeros(nat.NSCALARS, dtype=acc, device=dev)
        for k, g in enumerate((g0, g1, g2, g3)):
            if g is not None:
                gs[k] = g.to(acc)
        gseq_t = None
        if gseq is not None and gseq.numel():
            gseq_t = gseq.reshape(-1).to(acc).contiguous()
        _, _, views, _ = _views(kind, ck, ok, ak, mk)
        grad = torch.empty(B * T, dtype=acc, device=dev)
        nat.call(
            "rrl_policy_bwd", ctypes_ref(params), B, T, *views, nat.dtype_code(acc), ws.data_ptr(),
            gs.data_ptr(), nat.ptr(gseq_t), grad.data_ptr(), nat.stream_ptr(dev),
        )
        return None, grad.view(shape).to(dtype), None, None, None


def ctypes_ref(params: nat.RrlPolicyParams):
    return ctypes.byref(params)


def _objective(params: nat.RrlPolicyParams, cur: Tensor, old: Tensor, adv: Tensor, mask: Tensor):
    mask = _on_device(mask, cur)
    return _PolicyObjective.apply(params, cur, old, adv, mask)


def direct_double_sided_mask(ratios: Tensor, *, clip_low: float, clip_high: float) -> Tensor:
    """SAO's strict two-sided trust mask ``1 - clip_low < ratio < 1 + clip_high``
    (losses.py:104-124); boundary values are rejected."""

    if not ratios.is_floating_point():
        raise TypeError("ratios must be floating point")
    if not 0.0 <= clip_low < 1.0:
        raise ValueError("clip_low must be in [0, 1)")
    if clip_high < 0.0:
        raise ValueError("clip_high must be non-negative")
    dev = nat.require_device(ratios)
    r = ratios.contiguous()
    # torch compares a tensor with a Python scalar in the tensor's dtype
    lo = torch.tensor(1.0 - clip_low, dtype=ratios.dtype).item()
    hi = torch.tensor(1.0 + clip_high, dtype=ratios.dtype).item()
    out = torch.empty(ratios.shape, dtype=torch.bool, device=dev)
    nat.call("rrl_double_sided_mask", r.numel(), r.data_ptr(), nat.dtype_code(r.dtype), lo, hi,
             out.data_ptr(), nat.stream_ptr(dev))
    return out


def sao_policy_loss(
    current_logprobs: Tensor,
    rollout_logprobs: Tensor,
    advantages: Tensor,
    action_mask: Tensor,
    *,
    clip_low: float,
    clip_high: float,
    detach_ratio: bool = True,
    max_log_ratio: float = 20.0,
) -> SaoPolicyLossOutput:
    """SAO/DIS token objective (losses.py:127-203).

    Ratios outside the strict trust interval contribute a literal zero while
    the denominator stays all action tokens.  ``detach_ratio`` selects a
    stop-gradient importance weight (default) or the attached variant.
    """

    if not (
        current_logprobs.shape
        == rollout_logprobs.shape
        == advantages.shape
        == action_mask.shape
    ):
        raise ValueError("all tensors must have the same shape")
    if max_log_ratio <= 0.0:
        raise ValueError("max_log_ratio must be positive")
    if not 0.0 <= clip_low < 1.0:
        raise ValueError("clip_low must be in [0, 1)")
    if clip_high < 0.0:
        raise ValueError("clip_high must be non-negative")
    required_range = max(-math.log1p(-clip_low), math.log1p(clip_high))
    if max_log_ratio <= required_range:
        raise ValueError("max_log_ratio must exceed both trust-boundary log ratios")

    p = _params(nat.OBJ_SAO, clip_low=clip_low, clip_high=clip_high, max_log_ratio=max_log_ratio,
                detach_ratio=detach_ratio, mask_is_weight=False)
    obj, kl, rejected, ratio, _, trusted = _objective(
        p, current_logprobs, rollout_logprobs, advantages, action_mask
    )
    return SaoPolicyLossOutput(
        loss=-obj,
        objective=obj,
        approximate_kl=kl,
        rejected_fraction=rejected,
        mean_ratio=ratio,
        trusted_mask=trusted,
    )


def _check_rank2(name: str, current_logprobs: Tensor) -> None:
    if current_logprobs.ndim != 2:
        raise ValueError(f"{name} expects rank-2 [sequence, token] tensors")


def _check_float(*ts: Tensor) -> None:
    if not all(t.is_floating_point() for t in ts):
        raise TypeError("log-probabilities and advantages must be floating point")


def _check_clip_range(clip_low: float, clip_high: float, max_log_ratio: float) -> None:
    if not 0.0 <= clip_low < 1.0:
        raise ValueError("clip_low must be in [0, 1)")
    if clip_high < 0.0:
        raise ValueError("clip_high must be non-negative")
    if max_log_ratio <= 0.0:
        raise ValueError("max_log_ratio must be positive")
    required_range = max(-math.log1p(-clip_low), math.log1p(clip_high))
    if max_log_ratio <= required_range:
        raise ValueError("max_log_ratio must exceed both clip-boundary log ratios")


def gspo_policy_loss(
    current_logprobs: Tensor,
    rollout_logprobs: Tensor,
    sequence_advantages: Tensor,
    action_mask: Tensor,
    *,
    clip_low: float,
    clip_high: float,
    max_log_ratio: float = 20.0,
) -> GspoPolicyLossOutput:
    """GSPO sequence objective (losses.py:206-273): geometric-mean sequence
    ratios, clipped once per response, responses weighted equally."""

    _check_rank2("GSPO", current_logprobs)
    if not (current_logprobs.shape == rollout_logprobs.shape == action_mask.shape):
        raise ValueError("log-probability tensors and action_mask must match")
    if sequence_advantages.shape != current_logprobs.shape[:-1]:
        raise ValueError("sequence_advantages must have shape [sequence]")
    _check_float(current_logprobs, rollout_logprobs, sequence_advantages)
    _check_clip_range(clip_low, clip_high, max_log_ratio)

    p = _params(nat.OBJ_GSPO, clip_low=clip_low, clip_high=clip_high,
                max_log_ratio=max_log_ratio, mask_is_weight=False)
    obj, div, frac, mean_ratio, seq, _ = _objective(
        p, current_logprobs, rollout_logprobs, sequence_advantages, action_mask
    )
    return GspoPolicyLossOutput(
        loss=-obj,
        objective=obj,
        sequence_ratio_divergence=div,
        sequence_clip_fraction=frac,
        mean_sequence_ratio=mean_ratio,
        sequence_ratios=seq,
    )


def gspo_token_policy_loss(
    current_logprobs: Tensor,
    rollout_logprobs: Tensor,
    token_advantages: Tensor,
    action_mask: Tensor,
    *,
    clip_low: float,
    clip_high: float,
    max_log_ratio: float = 20.0,
) -> GspoPolicyLossOutput:
    """GSPO-token objective (losses.py:276-352): every token carries the
    sequence ratio numerically while its gradient flows through that token's
    own log-prob."""

    _check_rank2("GSPO-token", current_logprobs)
    if not (
        current_logprobs.shape
        == rollout_logprobs.shape
        == token_advantages.shape
        == action_mask.shape
    ):
        raise ValueError("all tensors must have the same shape")
    _check_float(current_logprobs, rollout_logprobs, token_advantages)
    _check_clip_range(clip_low, clip_high, max_log_ratio)

    p = _params(nat.OBJ_GSPO_TOKEN, clip_low=clip_low, clip_high=clip_high,
                max_log_ratio=max_log_ratio, mask_is_weight=False)
    obj, div, frac, mean_ratio, seq, _ = _objective(
        p, current_logprobs, rollout_logprobs, token_advantages, action_mask
    )
    return GspoPolicyLossOutput(
        loss=-obj,
        objective=obj,
        sequence_ratio_divergence=div,
        sequence_clip_fraction=frac,
        mean_sequence_ratio=mean_ratio,
        sequence_ratios=seq,
    )


def _check_sapo(current_logprobs, rollout_logprobs, token_advantages, action_mask,
                tau_positive, tau_negative, max_log_ratio) -> None:
    _check_rank2("SAPO", current_logprobs)
    if not (
        current_logprobs.shape
        == rollout_logprobs.shape
        == token_advantages.shape
        == action_mask.shape
    ):
        raise ValueError("all tensors must have the same shape")
    _check_float(current_logprobs, rollout_logprobs, token_advantages)
    if tau_positive <= 0.0 or tau_negative <= 0.0:
        raise ValueError("SAPO temperatures must be positive")
    if max_log_ratio <= 0.0:
        raise ValueError("max_log_ratio must be positive")


def sapo_policy_loss(
    current_logprobs: Tensor,
    rollout_logprobs: Tensor,
    token_advantages: Tensor,
    action_mask: Tensor,
    *,
    tau_positive: float = 1.0,
    tau_negative: float = 1.05,
    max_log_ratio: float = 20.0,
) -> SapoPolicyLossOutput:
    """SAPO smooth surrogate ``(4/tau) sigmoid(tau (ratio - 1)) A`` (losses.py:355-423),
    averaged within each response and then over responses."""

    _check_sapo(current_logprobs, rollout_logprobs, token_advantages, action_mask,
                tau_positive, tau_negative, max_log_ratio)
    p = _params(nat.OBJ_SAPO, max_log_ratio=max_log_ratio, tau_positive=tau_positive,
                tau_negative=tau_negative, mask_is_weight=False)
    obj, kl, ratio, gate, _, _ = _objective(
        p, current_logprobs, rollout_logprobs, token_advantages, action_mask
    )
    return SapoPolicyLossOutput(
        loss=-obj,
        objective=obj,
        approximate_kl=kl,
        mean_ratio=ratio,
        mean_gradient_gate=gate,
    )


def _check_clipped(current_logprobs, old_logprobs, advantages, action_mask, clip_low, clip_high,
                   max_log_ratio) -> float:
    if not (
        current_logprobs.shape
        == old_logprobs.shape
        == advantages.shape
        == action_mask.shape
    ):
        raise ValueError("all tensors must have the same shape")
    return _check_clip_params(clip_low, clip_high, max_log_ratio)


def _check_clip_params(clip_low, clip_high, max_log_ratio) -> float:
    if clip_low < 0:
        raise ValueError("clip_low must be non-negative")
    if clip_high is None:
        clip_high = clip_low
    if clip_high < 0:
        raise ValueError("clip_high must be non-negative")
    if max_log_ratio <= 0:
        raise ValueError("max_log_ratio must be positive")
    return clip_high


def clipped_policy_loss(
    current_logprobs: Tensor,
    old_logprobs: Tensor,
    advantages: Tensor,
    action_mask: Tensor,
    *,
    clip_low: float = 0.2,
    clip_high: Optional[float] = None,
    max_log_ratio: float = 20.0,
) -> PolicyLossOutput:
    """Globally token-normalized PPO/GRPO clipped loss (losses.py:426-486):
    ``-sum(m * min(rho A, clip(rho) A)) / sum(m)``."""

    clip_high = _check_clipped(current_logprobs, old_logprobs, advantages, action_mask, clip_low,
                               clip_high, max_log_ratio)
    p = _params(nat.OBJ_PPO, clip_low=clip_low, clip_high=clip_high,
                max_log_ratio=max_log_ratio, mask_is_weight=True)
    obj, kl, frac, ratio, _, _ = _objective(p, current_logprobs, old_logprobs, advantages,
                                            action_mask)
    return PolicyLossOutput(
        loss=-obj,
        objective=obj,
        approximate_kl=kl,
        clip_fraction=frac,
        mean_ratio=ratio,
    )


# ---------------------------------------------------------------------------
# a9: sequence_log_ratio
# ---------------------------------------------------------------------------


class _SequenceLogRatio(torch.autograd.Function):
    @staticmethod
    def forward(ctx, cur: Tensor, old: Tensor, mask: Tensor, normalize: bool) -> Tensor:
        dev = nat.require_device(cur, old, mask)
        B, T = cur.shape
        cv, _ = nat.rows_view(cur, B, T)
        ov, _ = nat.rows_view(old, B, T)
        mv, mk = nat.rows_view(mask, B, T)
        acc = nat.acc_dtype(cur.dtype, old.dtype)
        out = torch.empty(B, dtype=acc, device=dev)
        counts = torch.empty(B, dtype=acc, device=dev)
        status = nat.new_status(dev)
        nat.call("rrl_sequence_log_ratio_fwd", B, T, cv, ov, mv, int(normalize),
                 nat.dtype_code(acc), out.data_ptr(), counts.data_ptr(), status.data_ptr(),
                 nat.stream_ptr(dev))
        if B and nat.read_status(status) & nat.FLAG_EMPTY_ROW:
            raise ValueError("every sequence needs at least one action token")
        ctx.save_for_backward(mk, counts)
        ctx.meta = (B, T, acc, normalize, cur.dtype)
        ctx.set_materialize_grads(False)
        return out.to(cur.dtype)

    @staticmethod
    def backward(ctx, grad):
        if grad is None or not ctx.needs_input_grad[0]:
            return None, None, None, None
        mk, counts = ctx.saved_tensors
        B, T, acc, normalize, dtype = ctx.meta
        mv, _ = nat.rows_view(mk, B, T)
        g = grad.reshape(-1).to(acc).contiguous()
        gc = torch.empty(B * T, dtype=acc, device=counts.device)
        nat.call("rrl_sequence_log_ratio_bwd", B, T, mv, int(normalize), nat.dtype_code(acc),
                 counts.data_ptr(), g.data_ptr(), gc.data_ptr(), nat.stream_ptr(counts.device))
        return gc.view(B, T).to(dtype), None, None, None


def sequence_log_ratio(
    current_logprobs: Tensor,
    old_logprobs: Tensor,
    action_mask: Tensor,
    *,
    length_normalize: bool = True,
) -> Tensor:
    """Per-sequence sum (or mean) of token log-ratios (losses.py:489-512)."""

    if current_logprobs.ndim != 2:
        raise ValueError("sequence_log_ratio expects rank-2 tensors")
    if not (current_logprobs.shape == old_logprobs.shape == action_mask.shape):
        raise ValueError("all tensors must have the same shape")
    return _SequenceLogRatio.apply(current_logprobs, old_logprobs.detach(),
                                   _on_device(action_mask, current_logprobs),
                                   bool(length_normalize))


# ---------------------------------------------------------------------------
# Single pass: logits -> log-prob -> token-local objective -> dlogits
# ---------------------------------------------------------------------------

_OBJECTIVES = {
    "clipped": nat.OBJ_PPO,
    "ppo": nat.OBJ_PPO,
    "grpo": nat.OBJ_PPO,
    "sao": nat.OBJ_SAO,
    "sapo": nat.OBJ_SAPO,
    "gspo": nat.OBJ_GSPO,
    "gspo_token": nat.OBJ_GSPO_TOKEN,
}


def _token_local_params(kind: int, prefix, old_logprobs: Tensor, advantages: Tensor,
                       action_mask: Tensor, *, clip_low: float, clip_high: Optional[float],
                       max_log_ratio: float, detach_ratio: bool, tau_positive: float,
                       tau_negative: float) -> nat.RrlPolicyParams:
    """Validate a token-local objective's arguments (the checks and messages of
    clipped_policy_loss, sao_policy_loss and sapo_policy_loss) and pack its
    kernel parameters."""

    if kind == nat.OBJ_PPO:
        if not (prefix == old_logprobs.shape == advantages.shape == action_mask.shape):
            raise ValueError("all tensors must have the same shape")
        clip_high = _check_clip_params(clip_low, clip_high, max_log_ratio)
        p = _params(kind, clip_low=clip_low, clip_high=clip_high, max_log_ratio=max_log_ratio,
                    mask_is_weight=True)
    elif kind == nat.OBJ_SAO:
        if clip_high is None:
            raise TypeError("sao objective needs clip_high")
        if not (prefix == old_logprobs.shape == advantages.shape == action_mask.shape):
            raise ValueError("all tensors must have the same shape")
        if max_log_ratio <= 0.0:
            raise ValueError("max_log_ratio must be positive")
        _check_clip_range(clip_low, clip_high, max_log_ratio)
        p = _params(kind, clip_low=clip_low, clip_high=clip_high, max_log_ratio=max_log_ratio,
                    detach_ratio=detach_ratio, mask_is_weight=False)
    else:
        if len(prefix) != 2:
            raise ValueError("SAPO expects rank-2 [sequence, token] tensors")
        if not (prefix == old_logprobs.shape == advantages.shape == action_mask.shape):
            raise ValueError("all tensors must have the same shape")
        _check_float(old_logprobs, advantages)
        if tau_positive <= 0.0 or tau_negative <= 0.0:
            raise ValueError("SAPO temperatures must be positive")
        if max_log_ratio <= 0.0:
            raise ValueError("max_log_ratio must be positive")
        p = _params(kind, max_log_ratio=max_log_ratio, tau_positive=tau_positive,
                    tau_negative=tau_negative, mask_is_weight=False)

    return p


def _token_local_output(kind: int, obj: Tensor, d1: Tensor, d2: Tensor, d3: Tensor,
                        trusted: Tensor):
    """The output record of the token-local objective ``kind``."""

    if kind == nat.OBJ_PPO:
        return PolicyLossOutput(loss=-obj, objective=obj, approximate_kl=d1, clip_fraction=d2,
                                mean_ratio=d3)
    if kind == nat.OBJ_SAO:
        return SaoPolicyLossOutput(loss=-obj, objective=obj, approximate_kl=d1,
                                   rejected_fraction=d2, mean_ratio=d3, trusted_mask=trusted)
    return SapoPolicyLossOutput(loss=-obj, objective=obj, approximate_kl=d1, mean_ratio=d2,
                                mean_gradient_gate=d3)


class _FusedPolicy(torch.autograd.Function):
    """One sweep per logits row: log-prob, d(-objective)/d logp, dlogits.

    Forward stores dlogits for an upstream d loss = 1; backward rescales it on
    the device when autograd hands a different scale, and recomputes from the
    logits when diagnostics also receive gradients.
    """

    @staticmethod
    def forward(ctx, params: nat.RrlPolicyParams, inplace: bool, logits: Tensor,
                target_ids: Tensor, old: Tensor, adv: Tensor, mask: Tensor):
        kind = params.kind
        dev = nat.require_device(logits, target_ids, old, adv, mask)
        x, B, T, V, s_b, s_t = nat.logits_rows(logits)
        if inplace and x.data_ptr() != logits.data_ptr():
            raise RuntimeError("inplace=True needs logits whose rows can be addressed in place")
        tview, tkeep = nat.rows_view(target_ids, B, T)
        ov, ok = nat.rows_view(old, B, T)
        av, ak = nat.rows_view(adv, B, T)
        mv, mk = nat.rows_view(mask, B, T)
        acc = nat.acc_dtype(logits.dtype)
        acc_code = nat.dtype_code(acc)
        stream = nat.stream_ptr(dev)
        ws = torch.empty(nat.lib().rrl_policy_workspace_bytes(B, acc_code), dtype=torch.uint8,
                         device=dev)
        coef = torch.empty(B, dtype=acc, device=dev)
        records = torch.empty(nat.lib().rrl_fused_records_bytes(B, T), dtype=torch.uint8,
                              device=dev)
        logp = torch.empty(B * T, dtype=acc, device=dev)
        lse = torch.empty(B * T, dtype=acc, device=dev)
        if inplace:
            dl, d_b, d_t = x, s_b, s_t
        else:
            dl = torch.empty((B, T, V), dtype=logits.dtype, device=dev)
            d_b, d_t = T * V, V
        scal = torch.empty(nat.NSCALARS, dtype=acc, device=dev)
        trusted = torch.empty(B * T if kind == nat.OBJ_SAO else 0, dtype=torch.bool, device=dev)
        lview = nat.RrlView(logp.data_ptr(), acc_code, T, 1)

        early = _check_before_sweep(logits, inplace)
        rerun = _rerun_on_device(logits, inplace)

        def run(p):
            status = nat.new_status(dev)
            pref = ctypes_ref(p)
            nat.call("rrl_policy_row_coef", pref, B, T, mv, acc_code, coef.data_ptr(),
                     ws.data_ptr(), status.data_ptr(), stream)
            if early:
                nat.call("rrl_check_targets", pref, B, T, V, tview, status.data_ptr(), stream)
                _raise_flags(nat.read_status(status), kind)
            for q in (pref, ctypes_ref(_rerun_params(p))) if rerun else (pref,):
                nat.call("rrl_fused_logprob_policy", q, x.data_ptr(), nat.dtype_code(x.dtype),
                         B, T, V, s_b, s_t, tview, ov, av, mv, coef.data_ptr(),
                         records.data_ptr(), logp.data_ptr(), lse.data_ptr(), dl.data_ptr(),
                         nat.dtype_code(logits.dtype), d_b, d_t, status.data_ptr(), stream,
                         timed=q is pref)
            nat.call("rrl_policy_fwd", pref, B, T, lview, ov, av, mv, acc_code, ws.data_ptr(),
                     scal.data_ptr(), None, nat.ptr(trusted) if trusted.numel() else None,
                     status.data_ptr(), stream)
            return 0 if early else nat.read_status(status)

        flags = run(params)
        if flags & nat.FLAG_FAST_RANGE:
            # A row's log-sum-exp lies beyond the register-resident 16-bit kernel's exponent
            # range (logits near the format's maximum): redo the call on the
            # generic row kernel.
            if inplace:
                raise RuntimeError(
                    "fused_policy_loss(inplace=True): logits beyond +-2e38 need the generic "
                    "kernel, which cannot rerun over overwritten logits; call with inplace=False"
                )
            generic = nat.RrlPolicyParams.from_buffer_copy(params)
            generic.flags |= nat.POLICY_GENERIC
            flags = run(generic)
        _raise_flags(flags, kind)

        ctx.params = params
        ctx.inplace = inplace
        ctx.dl = dl
        ctx.meta = (B, T, V, s_b, s_t, d_b, d_t, acc, tuple(logits.shape), logits.dtype)
        ctx.save_for_backward(x if not inplace else lse, tkeep, ok, ak, mk, lse, logp, ws)
        ctx.set_materialize_grads(False)
        dts = _scalar_dtypes(kind, logp, old, adv)
        outs = [scal[k].to(dts[k], copy=True) for k in range(4)]
        logp_out = logp.view(logits.shape[:-1])
        trusted_out = trusted.view(logits.shape[:-1]) if kind == nat.OBJ_SAO else trusted
        if kind in (nat.OBJ_PPO, nat.OBJ_SAO):
            ctx.mark_non_differentiable(outs[2], logp_out, trusted_out)
        else:
            ctx.mark_non_differentiable(logp_out, trusted_out)
        return outs[0], outs[1], outs[2], outs[3], logp_out, trusted_out

    @staticmethod
    def backward(ctx, g0, g1, g2, g3, _glogp, _gtrusted):
        nones = (None, None)
        if not ctx.needs_input_grad[2]:
            return (*nones, None, None, None, None, None)
        B, T, V, s_b, s_t, d_b, d_t, acc, shape, dtype = ctx.meta
        params = ctx.params
        saved = ctx.saved_tensors
        x, tkeep, ok, ak, mk, lse, logp, ws = saved
        dev = lse.device
        stream = nat.stream_ptr(dev)
        dl = ctx.dl
        extra = any(g is not None for g in (g1, g3)) or (
            params.kind == nat.OBJ_SAPO and g2 is not None
        )
        if dl is not None and not extra:
            scale = (-g0).reshape(1).to(acc) if g0 is not None else torch.zeros(1, dtype=acc,
                                                                                 device=dev)
            nat.call("rrl_scale_rows", dl.data_ptr(), nat.dtype_code(dtype), B, T, V, d_b, d_t,
                     scale.data_ptr(), nat.dtype_code(acc), 1.0, stream)
            ctx.dl = None
            return (*nones, dl.view(shape), None, None, None, None)
        if ctx.inplace:
            raise RuntimeError(
                "fused_policy_loss(inplace=True) overwrote the logits; only loss.backward() "
                "once is supported"
            )
        # General case: full d/d logp from every differentiated output, then
        # one backward sweep over the logits.
        gs = torch.zeros(nat.NSCALARS, dtype=acc, device=dev)
        for k, g in enumerate((g0, g1, g2, g3)):
            if g is not None:
                gs[k] = g.to(acc)
        lview = nat.RrlView(logp.data_ptr(), nat.dtype_code(acc), T, 1)
        ov, _ = nat.rows_view(ok, B, T)
        av, _ = nat.rows_view(ak, B, T)
        mv, _ = nat.rows_view(mk, B, T)
        g = torch.empty(B * T, dtype=acc, device=dev)
        pref = ctypes_ref(params)
        nat.call("rrl_policy_bwd", pref, B, T, lview, ov, av, mv, nat.dtype_code(acc),
                 ws.data_ptr(), gs.data_ptr(), None, g.data_ptr(), stream)
        out = dl if dl is not None else torch.empty((B, T, V), dtype=dtype, device=dev)
        tview, _ = nat.rows_view(tkeep, B, T)
        nat.call("rrl_logprob_bwd", x.data_ptr(), nat.dtype_code(x.dtype), B, T, V, s_b, s_t,
                 tview, lse.data_ptr(), logp.data_ptr(), g.data_ptr(), out.data_ptr(),
                 nat.dtype_code(dtype), T * V, V, 0, stream)
        ctx.dl = None
        return (*nones, out.view(shape), None, None, None, None)


def fused_policy_loss(
    logits: Tensor,
    target_ids: Tensor,
    old_logprobs: Tensor,
    advantages: Tensor,
    action_mask: Tensor,
    *,
    objective: str = "clipped",
    clip_low: float = 0.2,
    clip_high: Optional[float] = None,
    max_log_ratio: float = 20.0,
    detach_ratio: bool = True,
    tau_positive: float = 1.0,
    tau_negative: float = 1.05,
    inplace: bool = False,
    return_logprobs: bool = False,
    skip_masked_rows: bool = False,
):
    """``objective(gather_token_logprobs(logits, target_ids), ...)`` in one sweep.

    Equal to composing :func:`gather_token_logprobs` with the named objective
    (``"clipped"``/``"ppo"``/``"grpo"``, ``"sao"``, ``"sapo"``, ``"gspo"``,
    ``"gspo_token"``) and returns that objective's output record, with the
    loss differentiable into ``logits``.  For the token-local objectives the
    forward streams each logits row once and writes dlogits then and there
    (read logits once, write dlogits once); GSPO needs every token's log-prob
    before any gradient and runs as the two-kernel composition.  GSPO takes
    ``advantages`` of shape ``[sequence]``.

    ``inplace=True`` writes dlogits over the logits (halves the memory of the
    step; the logits are destroyed).  ``return_logprobs=True`` returns
    ``(output, logprobs)``.

    ``skip_masked_rows=True`` (without ``return_logprobs``) never reads the
    logits of tokens whose mask weight is exactly 0: their dlogits rows are
    written as zeros (GSPO: its forward sweep skips them and its backward
    writes their zero-gradient rows unread).  For finite logits the loss and
    dlogits are bit-identical to the default; the one difference is that a
    NaN/inf logit at a masked position no longer turns the loss into NaN, as
    ``0 * NaN`` does in the reference's masked mean.
    """

    if objective not in _OBJECTIVES:
        raise ValueError(f"unknown objective {objective!r}; expected one of {sorted(_OBJECTIVES)}")
    kind = _OBJECTIVES[objective]
    if logits.ndim < 2:
        raise ValueError("logits must include positions and vocabulary")
    if logits.shape[:-1] != target_ids.shape:
        raise ValueError(
            f"target shape {target_ids.shape} must match logits prefix {logits.shape[:-1]}"
        )
    if target_ids.dtype not in (torch.int32, torch.int64):
        raise TypeError("target_ids must be an integer tensor")

    if skip_masked_rows and return_logprobs:
        raise ValueError("skip_masked_rows=True leaves masked log-probs uncomputed; "
                         "it cannot be combined with return_logprobs=True")
    if kind in (nat.OBJ_GSPO, nat.OBJ_GSPO_TOKEN):
        if inplace:
            raise ValueError("inplace=True applies to the single-sweep objectives only")
        # GSPO needs every token's log-prob before any gradient: a forward
        # sweep, then the objective, then a backward sweep that reuses the
        # forward's log-sum-exp and writes rows with a zero gradient unread.
        # With skip_masked_rows the forward does not read tokens whose mask
        # is 0: they enter the sequence log-ratio only times their zero mask.
        if skip_masked_rows:
            mask_dev = _on_device(action_mask, logits)
            if mask_dev.shape != target_ids.shape:
                mask_dev = mask_dev.expand(target_ids.shape)
            logp = _TokenLogprobs.apply(logits, target_ids, mask_dev)
        else:
            logp = gather_token_logprobs(logits, target_ids)
        fn = gspo_policy_loss if kind == nat.OBJ_GSPO else gspo_token_policy_loss
        out = fn(logp, old_logprobs, advantages, action_mask, clip_low=clip_low,
                 clip_high=clip_low if clip_high is None else clip_high,
                 max_log_ratio=max_log_ratio)
        return (out, _cfg.as_reference_dtype(logp.detach(), logits)) if return_logprobs else out

    p = _token_local_params(kind, logits.shape[:-1], old_logprobs, advantages, action_mask,
                            clip_low=clip_low, clip_high=clip_high,
                            max_log_ratio=max_log_ratio, detach_ratio=detach_ratio,
                            tau_positive=tau_positive, tau_negative=tau_negative)
    if skip_masked_rows:
        p.flags |= nat.POLICY_SKIP_MASKED
    mask = _on_device(action_mask, logits)
    obj, d1, d2, d3, logp, trusted = _FusedPolicy.apply(p, bool(inplace), logits, target_ids,
                                                        old_logprobs, advantages, mask)
    out = _token_local_output(kind, obj, d1, d2, d3, trusted)
    return (out, _cfg.as_reference_dtype(logp, logits)) if return_logprobs else out

