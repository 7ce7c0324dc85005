"""PyTorch-CPU restatement of the RoseRLHF hot path — TEST INFRASTRUCTURE ONLY.

Each function restates one reference function (cited file:line under
rosellm/roserlhf/) from its mathematical contract: same inputs, outputs, mask
semantics, threshold rules and error conditions, evaluated with ordinary
PyTorch CPU ops so that autograd supplies the gradients exactly as in the
reference's own composition.  bf16 inputs are evaluated on their exact float32
upcast (the parity contract of the GPU kernels).

Pinned by: the reference's known-answer tests (tests/golden), float64 brute
force (oracle/brute.py), closed-form gradients, and invariants — see
tests/test_oracle.py.  ``masked_whiten`` has no reference counterpart: parity
unpinned (closed form and invariants only).  ``nll_loss`` / ``sft_step`` (the
SFT loss of rosetrainer/model.py:643-649) are pinned by torch's own
F.cross_entropy in float64 and by the scalar loops of oracle/brute.py.
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import torch
import torch.nn.functional as F
from torch import Tensor

# ---------------------------------------------------------------------------
# log-probs (losses.py:14-38)
# ---------------------------------------------------------------------------


def token_logprobs(logits: Tensor, targets: Tensor, *, exact: bool = False) -> Tensor:
    """log p(target) per position: the vocabulary log-softmax, then a gather.

    ``exact=True`` evaluates on the float64 upcast of the logits (exact for
    every float dtype), which is the value a float32 kernel is held to.
    """

    if exact:
        x = logits.double()
    else:
        x = logits.float() if logits.dtype in (torch.bfloat16, torch.float16) else logits
    logsm = F.log_softmax(x, dim=-1)
    return torch.take_along_dim(logsm, targets.long().unsqueeze(-1), dim=-1).squeeze(-1)


# ---------------------------------------------------------------------------
# objectives (losses.py:41-512)
# ---------------------------------------------------------------------------


def weighted_average(values: Tensor, mask: Tensor) -> Tensor:
    """sum(values * w) / sum(w) with w = mask in the value dtype (losses.py:41-50)."""

    w = mask.to(values.dtype)
    total_w = w.sum()
    if total_w.item() == 0:
        raise ValueError("cannot reduce an empty mask")
    return (values * w).sum() / total_w


def _ratio(cur: Tensor, old: Tensor, bound: float) -> Tuple[Tensor, Tensor]:
    """(ratio, clamped log-ratio) with the log-ratio clamped to +-bound."""

    lr = (cur - old.detach()).clamp(-bound, bound)
    return lr.exp(), lr


def ppo_clip(cur: Tensor, old: Tensor, adv: Tensor, mask: Tensor, *, clip_low: float = 0.2,
             clip_high: Optional[float] = None, max_log_ratio: float = 20.0) -> Dict[str, Tensor]:
    """Globally token-normalized PPO/GRPO clip (losses.py:426-486)."""

    hi_eps = clip_low if clip_high is None else clip_high
    rho, lr = _ratio(cur, old, max_log_ratio)
    a = adv.detach()
    per_token = torch.minimum(rho * a, rho.clamp(1.0 - clip_low, 1.0 + hi_eps) * a)
    obj = weighted_average(per_token, mask)
    outside = (rho < 1.0 - clip_low) | (rho > 1.0 + hi_eps)
    return {
        "loss": -obj,
        "objective": obj,
        "approximate_kl": weighted_average(rho - 1.0 - lr, mask),
        "clip_fraction": weighted_average(outside.to(rho.dtype), mask),
        "mean_ratio": weighted_average(rho, mask),
    }


def strict_trust(ratios: Tensor, *, clip_low: float, clip_high: float) -> Tensor:
    """DIS trust mask, open interval (losses.py:104-124)."""

    return (ratios > 1.0 - clip_low) & (ratios < 1.0 + clip_high)


def sao(cur: Tensor, rollout: Tensor, adv: Tensor, mask: Tensor, *, clip_low: float,
        clip_high: float, detach_ratio: bool = True, max_log_ratio: float = 20.0
        ) -> Dict[str, Tensor]:
    """SAO/DIS objective (losses.py:127-203)."""

    rho, lr = _ratio(cur, rollout, max_log_ratio)
    keep = strict_trust(rho, clip_low=clip_low, clip_high=clip_high)
    m = mask.to(torch.bool)
    iw = rho.detach() if detach_ratio else rho
    contrib = torch.where(keep, iw * adv.detach() * cur, torch.zeros_like(cur))
    obj = weighted_average(contrib, m)
    return {
        "loss": -obj,
        "objective": obj,
        "approximate_kl": weighted_average(rho - 1.0 - lr, m),
        "rejected_fraction": weighted_average((~keep).to(rho.dtype), m),
        "mean_ratio": weighted_average(rho, m),
        "trusted_mask": keep & m,
    }


def _row_counts(mask: Tensor) -> Tuple[Tensor, Tensor]:
    m = mask.to(torch.bool)
    n = m.sum(dim=-1)
    if (n == 0).any():
        raise ValueError("every sequence needs at least one action token")
    return m, n


def _sequence_ratio(cur: Tensor, rollout: Tensor, m: Tensor, n: Tensor, bound: float):
    w = m.to(cur.dtype)
    mean_lr = ((cur - rollout.detach()) * w).sum(dim=-1) / n
    safe = mean_lr.clamp(-bound, bound)
    return safe.exp(), safe, w


def gspo(cur: Tensor, rollout: Tensor, seq_adv: Tensor, mask: Tensor, *, clip_low: float,
         clip_high: float, max_log_ratio: float = 20.0) -> Dict[str, Tensor]:
    """GSPO sequence-level objective (losses.py:206-273)."""

    m, n = _row_counts(mask)
    s, safe, _ = _sequence_ratio(cur, rollout, m, n, max_log_ratio)
    a = seq_adv.detach()
    obj = torch.minimum(s * a, s.clamp(1.0 - clip_low, 1.0 + clip_high) * a).mean()
    out_of_band = (s < 1.0 - clip_low) | (s > 1.0 + clip_high)
    return {
        "loss": -obj,
        "objective": obj,
        "sequence_ratio_divergence": (s - 1.0 - safe).mean(),
        "sequence_clip_fraction": out_of_band.to(s.dtype).mean(),
        "mean_sequence_ratio": s.mean(),
        "sequence_ratios": s,
    }


def gspo_token(cur: Tensor, rollout: Tensor, tok_adv: Tensor, mask: Tensor, *, clip_low: float,
               clip_high: float, max_log_ratio: float = 20.0) -> Dict[str, Tensor]:
    """GSPO-token with the stop-gradient carrier exp(l - sg(l)) (losses.py:276-352)."""

    m, n = _row_counts(mask)
    s, safe, w = _sequence_ratio(cur, rollout, m, n, max_log_ratio)
    tok_ratio = s.detach().unsqueeze(-1) * (cur - cur.detach()).exp()
    a = tok_adv.detach()
    per_tok = torch.minimum(tok_ratio * a, tok_ratio.clamp(1.0 - clip_low, 1.0 + clip_high) * a)
    obj = ((per_tok * w).sum(dim=-1) / n).mean()
    out_of_band = (s < 1.0 - clip_low) | (s > 1.0 + clip_high)
    return {
        "loss": -obj,
        "objective": obj,
        "sequence_ratio_divergence": (s - 1.0 - safe).mean(),
        "sequence_clip_fraction": out_of_band.to(s.dtype).mean(),
        "mean_sequence_ratio": s.mean(),
        "sequence_ratios": s,
    }


def sapo(cur: Tensor, rollout: Tensor, tok_adv: Tensor, mask: Tensor, *,
         tau_positive: float = 1.0, tau_negative: float = 1.05, max_log_ratio: float = 20.0
         ) -> Dict[str, Tensor]:
    """SAPO soft-gated objective (losses.py:355-423)."""

    m, n = _row_counts(mask)
    w = m.to(cur.dtype)
    rho, lr = _ratio(cur, rollout, max_log_ratio)
    a = tok_adv.detach()
    tau = torch.where(a > 0.0, torch.full_like(a, tau_positive), torch.full_like(a, tau_negative))
    p = torch.sigmoid(tau * (rho - 1.0))
    soft = (4.0 / tau) * p * a

    def seq_avg(v: Tensor) -> Tensor:
        return ((v * w).sum(dim=-1) / n).mean()

    obj = seq_avg(soft)
    return {
        "loss": -obj,
        "objective": obj,
        "approximate_kl": seq_avg(rho - 1.0 - lr),
        "mean_ratio": seq_avg(rho),
        "mean_gradient_gate": seq_avg(4.0 * p * (1.0 - p)),
    }


def sequence_log_ratio(cur: Tensor, old: Tensor, mask: Tensor, *, length_normalize: bool = True
                       ) -> Tensor:
    """Per-row sum of w * (cur - old), optionally / sum(w) (losses.py:489-512)."""

    w = mask.to(cur.dtype)
    n = w.sum(dim=-1)
    if (n == 0).any():
        raise ValueError("every sequence needs at least one action token")
    total = ((cur - old.detach()) * w).sum(dim=-1)
    return total / n if length_normalize else total


# ---------------------------------------------------------------------------
# estimators (advantages.py:17-290)
# ---------------------------------------------------------------------------


def _flag(mask: Optional[Tensor], like: Tensor, default: bool) -> Tensor:
    if mask is None:
        return torch.full(like.shape, default, dtype=torch.bool)
    return mask.to(torch.bool)


def returns_to_go(rewards: Tensor, *, gamma: float = 1.0, terminated: Optional[Tensor] = None,
                  valid_mask: Optional[Tensor] = None, bootstrap_value: Optional[Tensor] = None
                  ) -> Tensor:
    """Backward recursion R_t = r_t + gamma (1 - d_t) R_{t+1} on valid steps,
    padding carries R and outputs 0 (advantages.py:25-80)."""

    valid = _flag(valid_mask, rewards, True)
    done = _flag(terminated, rewards, False)
    carry = (torch.zeros(rewards.shape[:-1], dtype=rewards.dtype) if bootstrap_value is None
             else bootstrap_value.to(rewards.dtype).clone())
    out = torch.zeros_like(rewards)
    for t in reversed(range(rewards.shape[-1])):
        step = rewards[..., t] + gamma * (~done[..., t]).to(rewards.dtype) * carry
        carry = torch.where(valid[..., t], step, carry)
        out[..., t] = torch.where(valid[..., t], carry, torch.zeros_like(carry))
    return out


def gae(rewards: Tensor, values: Tensor, *, gamma: float = 1.0, gae_lambda: float = 1.0,
        terminated: Optional[Tensor] = None, valid_mask: Optional[Tensor] = None,
        bootstrap_value: Optional[Tensor] = None) -> Tuple[Tensor, Tensor]:
    """GAE with padding skipped and terminals cutting bootstrap and trace
    (advantages.py:83-142)."""

    valid = _flag(valid_mask, rewards, True)
    done = _flag(terminated, rewards, False)
    v_next = (torch.zeros(rewards.shape[:-1], dtype=values.dtype) if bootstrap_value is None
              else bootstrap_value.to(values.dtype).clone())
    a_next = torch.zeros_like(v_next)
    adv = torch.zeros_like(rewards)
    for t in reversed(range(rewards.shape[-1])):
        cont = (~done[..., t]).to(rewards.dtype)
        td = rewards[..., t] + gamma * cont * v_next - values[..., t]
        a_t = torch.where(valid[..., t], td + gamma * gae_lambda * cont * a_next,
                          torch.zeros_like(td))
        adv[..., t] = a_t
        v_next = torch.where(valid[..., t], values[..., t], v_next)
        a_next = torch.where(valid[..., t], a_t, a_next)
    return adv, torch.where(valid, adv + values, torch.zeros_like(values))


def skip_observation_gae(rewards: Tensor, action_end_values: Tensor, next_action_values: Tensor,
                         *, gamma: float = 1.0, gae_lambda: float = 1.0,
                         terminated: Optional[Tensor] = None,
                         valid_mask: Optional[Tensor] = None) -> Tuple[Tensor, Tensor]:
    """Action-to-action GAE with explicit next-action values (advantages.py:145-217)."""

    valid = _flag(valid_mask, rewards, True)
    done = _flag(terminated, rewards, False)
    a_next = torch.zeros(rewards.shape[:-1], dtype=rewards.dtype)
    adv = torch.zeros_like(rewards)
    for i in reversed(range(rewards.shape[-1])):
        cont = (~done[..., i]).to(rewards.dtype)
        td = rewards[..., i] + gamma * cont * next_action_values[..., i] - action_end_values[..., i]
        a_i = torch.where(valid[..., i], td + gamma * gae_lambda * cont * a_next,
                          torch.zeros_like(td))
        adv[..., i] = a_i
        a_next = torch.where(valid[..., i], a_i, a_next)
    return adv, torch.where(valid, adv + action_end_values, torch.zeros_like(action_end_values))


def leave_one_out(rewards: Tensor, *, dim: int = -1) -> Tensor:
    """r_i minus the mean of the other group members (advantages.py:220-233)."""

    g = rewards.shape[dim]
    if g < 2:
        raise ValueError("leave-one-out advantages require group_size >= 2")
    others = (rewards.sum(dim=dim, keepdim=True) - rewards) / (g - 1)
    return rewards - others


def group_standardize(rewards: Tensor, *, dim: int = -1, eps: float = 1e-8) -> Tensor:
    """(r - mean) / max(std_pop, eps), zero where std_pop <= eps (advantages.py:236-258).

    A uniform group (max == min) has std 0 exactly, the contract the
    reference's docstring states (advantages.py:243-244).  torch's vectorised
    CPU ``std`` leaves a few 1e-8 on uniform groups of 8 or more non-dyadic
    values (e.g. 8 x 0.3 gives 2.98e-8 > eps = 1e-8, hence +-1 outputs); that
    rounding artefact is not reproduced.
    """

    if rewards.shape[dim] < 2:
        raise ValueError("group standardization requires group_size >= 2")
    mu = rewards.mean(dim=dim, keepdim=True)
    sd = rewards.std(dim=dim, unbiased=False, keepdim=True)
    uniform = rewards.amax(dim=dim, keepdim=True) == rewards.amin(dim=dim, keepdim=True)
    sd = torch.where(uniform, torch.zeros_like(sd), sd)
    z = (rewards - mu) / sd.clamp_min(eps)
    return torch.where(sd > eps, z, torch.zeros_like(z))


def turn_broadcast(turn_adv: Tensor, turn_ids: Tensor, mask: Tensor) -> Tensor:
    """out[b, t] = mask ? turn_adv[b, id] : 0 (advantages.py:261-290)."""

    m = mask.to(torch.bool)
    ids = turn_ids.long()
    bad = m & ((ids < 0) | (ids >= turn_adv.shape[1]))
    if bad.any():
        raise ValueError("an unmasked policy token has an invalid turn ID")
    picked = turn_adv.gather(1, ids.clamp(0, max(turn_adv.shape[1] - 1, 0)))
    return torch.where(m, picked, torch.zeros_like(picked))


def masked_whiten(values: Tensor, mask: Tensor, *, eps: float = 1e-8, shift_mean: bool = True
                  ) -> Tensor:
    """(x - mean_m) / (std_pop_m + eps) on masked tokens, 0 elsewhere.

    No reference function exists (parity unpinned); definition chosen for
    whitened PPO advantages.
    """

    m = mask.to(torch.bool)
    sel = values[m]
    if sel.numel() == 0:
        raise ValueError("cannot reduce an empty mask")
    mu = sel.mean()
    sd = ((sel - mu) ** 2).mean().sqrt()
    y = ((values - mu) if shift_mean else values) / (sd + eps)
    return torch.where(m, y, torch.zeros_like(y))


# ---------------------------------------------------------------------------
# compositions
# ---------------------------------------------------------------------------


def grpo_step(logits: Tensor, targets: Tensor, old: Tensor, adv: Tensor, mask: Tensor, *,
              clip_low: float, clip_high: Optional[float] = None,
              max_log_ratio: float = 20.0) -> Tuple[Dict[str, Tensor], Tensor, Tensor]:
    """log-softmax -> gather -> clipped objective -> autograd backward, the
    composition of examples/agentic_rl_toy.py:97-120 on given logits.

    Returns (objective outputs, log-probs, dlogits).  dlogits is in the dtype
    the objective was evaluated in (float32 for 16-bit logits).
    """

    x = logits.detach()
    x = (x.float() if x.dtype in (torch.bfloat16, torch.float16) else x.clone()).requires_grad_()
    lp = token_logprobs(x, targets)
    out = ppo_clip(lp, old, adv, mask, clip_low=clip_low, clip_high=clip_high,
                   max_log_ratio=max_log_ratio)
    out["loss"].backward()
    return out, lp.detach(), x.grad


def policy_step(kind: str, logits: Tensor, targets: Tensor, old: Tensor, adv: Tensor,
                mask: Tensor, *, exact: bool = False, **kw
                ) -> Tuple[Dict[str, Tensor], Tensor, Tensor]:
    """Like grpo_step for any objective name ('ppo', 'sao', 'gspo', 'gspo_token', 'sapo').

    ``exact=True`` runs the whole composition in float64 on exact upcasts of
    the inputs (the reference's math without float32 rounding).
    """

    fns = {"ppo": ppo_clip, "sao": sao, "gspo": gspo, "gspo_token": gspo_token, "sapo": sapo}
    x = logits.detach()
    if exact:
        x = x.double().requires_grad_()
        old, adv = old.double(), adv.double()
        if mask.is_floating_point():
            mask = mask.double()
    else:
        x = (x.float() if x.dtype in (torch.bfloat16, torch.float16) else x.clone())
        x.requires_grad_()
    lp = token_logprobs(x, targets)
    lp.retain_grad()
    out = fns[kind](lp, old, adv, mask, **kw)
    out["loss"].backward()
    out["dloss_dlogp"] = lp.grad.detach()
    return out, lp.detach(), x.grad


def lm_head_step(kind: str, hidden: Tensor, weight: Tensor, logits: Tensor, targets: Tensor,
                 old: Tensor, adv: Tensor, mask: Tensor, *, exact: bool = False, **kw
                 ) -> Tuple[Dict[str, Tensor], Tensor, Tensor, Tensor]:
    """policy_step behind the LM head: logits = hidden @ weight.T with no bias
    (rosetrainer/model.py:499,641; rosetrainer/qwen3.py:508,556), then the
    objective, then the linear map's backward: d hidden = dlogits @ weight,
    d weight = dlogits.T @ hidden (summed over every token).

    ``logits`` are the rounded products the kernels under test consumed (the
    product itself is the GEMM library's); pass the float64 product of
    ``hidden`` and ``weight`` to run the whole chain exactly.  With 16-bit
    logits the reference's autograd hands the linear map's backward a
    gradient in the logits dtype, so dlogits are rounded to it (round to
    nearest even) before the two products, as there.  Returns (objective
    outputs with the dlogits so used under "dlogits", log-probs, d hidden,
    d weight).
    """

    out, lp, dl = policy_step(kind, logits, targets, old, adv, mask, exact=exact, **kw)
    wide = torch.float64 if exact else torch.float32
    V, H = weight.shape
    if logits.dtype in (torch.bfloat16, torch.float16):
        dl = dl.to(logits.dtype)
    out["dlogits"] = dl
    d2 = dl.reshape(-1, V).to(wide)
    h2 = hidden.reshape(-1, H).to(wide)
    dh = (d2 @ weight.to(wide)).reshape(hidden.shape)
    dw = d2.t() @ h2
    return out, lp, dh, dw


# ---------------------------------------------------------------------------
# SFT next-token cross-entropy (rosetrainer/model.py:643-649,
# rosetrainer/qwen3.py:558-564)
# ---------------------------------------------------------------------------


def nll_loss(logits: Tensor, labels: Tensor, *, ignore_index: int = -100,
             reduction: str = "mean", exact: bool = False) -> Tensor:
    """F.cross_entropy(logits.view(-1, V), labels.view(-1)) restated from its
    definition: the vocabulary log-softmax, a gather at each label, and the
    negated mean (or sum) over the labels that differ from ``ignore_index``
    (the class dimension is last).  An ignored label is never gathered; the
    "mean" of no tokens is 0/0 = NaN.  Other ids outside [0, V) raise
    IndexError, as F.cross_entropy does."""

    V = logits.shape[-1]
    x = logits.reshape(-1, V)
    y = labels.reshape(-1).long()
    keep = y != ignore_index
    if bool(((y < 0) | (y >= V))[keep].any()):
        raise IndexError("Target is out of bounds")
    lp = token_logprobs(x, torch.where(keep, y, torch.zeros_like(y)), exact=exact)
    total = torch.where(keep, lp, torch.zeros_like(lp)).sum()
    if reduction == "sum":
        return -total
    return -(total / keep.sum().to(total.dtype))


def sft_step(logits: Tensor, labels: Tensor, *, causal: bool = True, ignore_index: int = -100,
             reduction: str = "mean", exact: bool = False) -> Tuple[Tensor, Tensor]:
    """The reference's LM loss and its gradient: with ``causal`` the shift of
    rosetrainer/model.py:644-645 (logits [B, T, V] at t score labels at t+1),
    then nll_loss, then autograd.  Returns (loss, dlogits of the full logits'
    shape; zero rows at the last position when causal).  16-bit logits are
    evaluated on their float32 upcast (float64 with ``exact``)."""

    x = logits.detach()
    wide = torch.float64 if exact else (
        torch.float32 if x.dtype in (torch.bfloat16, torch.float16) else x.dtype)
    x = x.to(wide).requires_grad_()
    if causal:
        loss = nll_loss(x[:, :-1], labels[:, 1:], ignore_index=ignore_index,
                        reduction=reduction)
    else:
        loss = nll_loss(x, labels, ignore_index=ignore_index, reduction=reduction)
    loss.backward()
    return loss.detach(), x.grad


def clip_bounds(clip_low: float, clip_high: float) -> Tuple[float, float]:
    """Both log-ratio boundaries of the clip band (used by validators)."""

    return -math.log1p(-clip_low), math.log1p(clip_high)
