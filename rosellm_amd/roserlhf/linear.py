"""Fused LM-head + token log-prob + policy objective, without the logits tensor.

The neighbour of the hot path on the producer side: the reference forms
``logits = lm_head(hidden)`` (``rosetrainer/model.py:499,641``,
``rosetrainer/qwen3.py:508,556``, no bias) and then calls
``gather_token_logprobs`` (``roserlhf/losses.py:14-38``) and an objective,
holding the whole ``[tokens, V]`` logits tensor (79.7 GB at 262,144 tokens x
151,936 vocab in bf16) plus its gradient.

Here the hidden x vocabulary product runs on the gfx950 matrix cores in
hand-written kernels (``csrc/lm_head.hip``) that never hold more than a
32 x 64 logits tile:

* the forward streams the vocabulary past 64-token blocks, keeping an online
  softmax per token, and forms in the same pass ``obar_n = sum_{v != a_n}
  p_nv W_v`` (an attention-shaped product with keys = values = the weight
  rows);
* ``dhidden_n = g_n ((1 - p_target) W[a_n] - obar_n)`` is then an elementwise
  kernel, with ``g = d loss / d logp`` from the objective's own backward;
* ``dW`` streams the tokens past 64-row blocks of the weight, recomputing each
  logits tile from the saved log-sum-exp (``dW_v = sum_n g_n ([v == a_n] -
  p_nv) hidden_n``), accumulating in float32 registers and writing once.

That is 4 x 2·N·H·V flops per step (the forward's two products and the dW
pass's two) and no HBM traffic proportional to N·V.  Any objective of the
package composes with it through autograd: the log-probs are an ordinary
differentiable tensor.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from .. import _native as nat
from .. import _config as _cfg
from . import losses as L

__all__ = ["fused_linear_policy_loss", "linear_token_logprobs"]

# Accepted for compatibility with callers that sized the logits they could
# afford; the matrix-core path never forms more than a 32 x 64 logits tile.
DEFAULT_ROW_BLOCK = 16384

# The softmax weights pass through the MFMA as 16-bit values: bfloat16 holds
# weights of order 1/V; float16's normal range stops at 6.1e-5.
_MFMA_DTYPES = (torch.bfloat16,)


def _prepare(hidden: Tensor, weight: Tensor, target_ids: Tensor):
    if hidden.ndim < 2:
        raise ValueError("hidden must include positions and the hidden dimension")
    if weight.ndim != 2 or weight.shape[1] != hidden.shape[-1]:
        raise ValueError(f"weight must be [vocab, {hidden.shape[-1]}], got {tuple(weight.shape)}")
    if hidden.dtype != weight.dtype:
        raise TypeError("hidden and weight must share a dtype")
    if hidden.dtype not in (torch.bfloat16, torch.float16, torch.float32, torch.float64):
        raise TypeError("hidden must be a floating point tensor")
    if hidden.shape[:-1] != target_ids.shape:
        raise ValueError(
            f"target shape {target_ids.shape} must match hidden prefix {hidden.shape[:-1]}")
    if target_ids.dtype not in (torch.int32, torch.int64):
        raise TypeError("target_ids must be an integer tensor")
    prefix = hidden.shape[:-1]
    B, T = (1, int(prefix[0])) if len(prefix) == 1 else nat.flatten_rows(prefix)
    return B, T


def _check_mfma(hidden: Tensor) -> None:
    H = hidden.shape[-1]
    if hidden.dtype not in _MFMA_DTYPES:
        raise TypeError("the matrix-core LM head takes bfloat16 hidden states and weights, "
                        f"got {hidden.dtype}")
    if H % 128 != 0 or not 128 <= H <= 1024:
        raise ValueError(f"the matrix-core LM head needs a hidden size that is a multiple of 128 "
                         f"in [128, 1024], got {H}")


def _rows2d(t: Tensor, n: int, h: int) -> Tensor:
    """[n, h] rows with one row stride (a multiple of 8 elements, 16-byte
    aligned base), copying only when the view has no such layout."""

    x = t.reshape(n, h)
    if (x.stride(-1) != 1 or x.stride(0) % 8 != 0 or x.stride(0) < h
            or x.data_ptr() % 16 != 0):
        x = x.contiguous()
    return x


def _targets_i32(target_ids: Tensor, n: int) -> Tensor:
    return target_ids.reshape(n).to(torch.int32).contiguous()


def lm_head_forward(h2: Tensor, w: Tensor, tgt32: Tensor, want_obar: bool, status: Tensor,
                    need: Optional[Tensor] = None
                    ) -> Tuple[Tensor, Tensor, Optional[Tensor], int]:
    """(lse, logp, obar, status flags): lse and logp float32 [N], obar float32
    [N, H] when ``want_obar`` (else None).  Reads the status word once (one
    host synchronisation).  If a token's logits leave the single pass's fixed
    reference range (flag LM_RANGE), the pass is redone around the exact
    log-sum-exp of a second, log-sum-exp-only pass.  ``need``: optional uint8
    [N]; 64-token blocks with no needed token skip obar (left unwritten)."""

    dev = h2.device
    N, H = h2.shape
    V = w.shape[0]
    dt = nat.dtype_code(h2.dtype)
    stream = nat.stream_ptr(dev)
    lse = torch.empty(N, dtype=torch.float32, device=dev)
    logp = torch.empty(N, dtype=torch.float32, device=dev)
    obar = torch.empty((N, H), dtype=torch.float32, device=dev) if want_obar else None
    need_p = nat.ptr(need) if (want_obar and need is not None) else None
    ws = None
    if need_p is not None:
        ws = torch.empty(nat.lib().rrl_lm_head_fwd_workspace_bytes(N), dtype=torch.uint8,
                         device=dev)
    nat.call("rrl_lm_head_fwd", h2.data_ptr(), w.data_ptr(), dt, N, H, V, h2.stride(0),
             w.stride(0), tgt32.data_ptr(), need_p, None, lse.data_ptr(), logp.data_ptr(),
             nat.ptr(obar), H, nat.ptr(ws), status.data_ptr(), stream)
    flags = nat.read_status(status)
    if flags & nat.FLAG_LM_RANGE and want_obar:
        # Exact log-sum-exp first, then the single pass around it.
        mref = torch.empty(N, dtype=torch.float32, device=dev)
        nat.call("rrl_lm_head_fwd", h2.data_ptr(), w.data_ptr(), dt, N, H, V, h2.stride(0),
                 w.stride(0), tgt32.data_ptr(), None, None, mref.data_ptr(), logp.data_ptr(),
                 None, H, None, status.data_ptr(), stream)
        nat.call("rrl_lm_head_fwd", h2.data_ptr(), w.data_ptr(), dt, N, H, V, h2.stride(0),
                 w.stride(0), tgt32.data_ptr(), need_p, mref.data_ptr(), lse.data_ptr(),
                 logp.data_ptr(), nat.ptr(obar), H, nat.ptr(ws), status.data_ptr(), stream)
        flags = nat.read_status(status) & ~nat.FLAG_LM_RANGE
    return lse, logp, obar, flags


def lm_head_backward(h2: Tensor, w: Tensor, tgt32: Tensor, lse: Tensor, logp: Tensor,
                     obar: Tensor, g: Tensor, need_h: bool, need_w: bool):
    """d hidden [N, H] and d weight [V, H] (both in the weight dtype) for
    g = d loss / d logp."""

    dev = h2.device
    N, H = h2.shape
    V = w.shape[0]
    dt = nat.dtype_code(h2.dtype)
    stream = nat.stream_ptr(dev)
    dh = dw = None
    if need_h:
        dh = torch.empty((N, H), dtype=h2.dtype, device=dev)
        nat.call("rrl_lm_head_dhidden", w.data_ptr(), dt, N, H, V, w.stride(0), tgt32.data_ptr(),
                 logp.data_ptr(), g.data_ptr(), obar.data_ptr(), H, dh.data_ptr(), H, stream)
    if need_w:
        dw = torch.empty((V, H), dtype=w.dtype, device=dev)
        rec = torch.empty(nat.lib().rrl_lm_head_dweight_workspace_bytes(N, H, V),
                          dtype=torch.uint8, device=dev)
        nat.call("rrl_lm_head_dweight", h2.data_ptr(), w.data_ptr(), dt, N, H, V, h2.stride(0),
                 w.stride(0), tgt32.data_ptr(), lse.data_ptr(), logp.data_ptr(), g.data_ptr(),
                 rec.data_ptr(), dw.data_ptr(), dt, H, stream)
    return dh, dw


class _LinearLogprobs(torch.autograd.Function):
    """log_softmax(hidden @ weight.T)[target] on the matrix cores; the forward
    keeps obar for d hidden, the backward recomputes logits tiles for d W.

    ``check``: the objective parameters whose target rule applies (any id
    outside [0, V) raises, as torch.gather does, except NLL's ignore_index,
    whose tokens get no target and log-prob 0)."""

    @staticmethod
    def forward(ctx, check: nat.RrlPolicyParams, hidden: Tensor, weight: Tensor,
                target_ids: Tensor, weight_mask: Optional[Tensor] = None,
                skip_masked: bool = False):
        dev = nat.require_device(hidden, weight, target_ids)
        B, T = _prepare(hidden, weight, target_ids)
        _check_mfma(hidden)
        N, H = B * T, hidden.shape[-1]
        V = weight.shape[0]
        h2 = _rows2d(hidden, N, H)
        w = _rows2d(weight, V, H)
        ids = target_ids
        if check.kind == nat.OBJ_NLL:
            ids = torch.where(target_ids == check.ignore_index, -1, target_ids)
        tgt32 = _targets_i32(ids, N)
        status = nat.new_status(dev)
        tv, _keep = nat.rows_view(target_ids.reshape(B, T), B, T)
        nat.call("rrl_check_targets", L.ctypes_ref(check), B, T, V, tv, status.data_ptr(),
                 nat.stream_ptr(dev))
        need = ctx.needs_input_grad[1] or ctx.needs_input_grad[2]
        # Tokens whose mask weight is zero get d loss / d logp = 0 from every
        # objective here, so their obar (the d hidden term) is never read;
        # with skip_masked their log-probs are not needed either (value 2: a
        # block of 64 such tokens is not computed, its log-probs are 0).
        need_rows = None
        if need and weight_mask is not None:
            live = weight_mask.reshape(N) != 0
            if skip_masked:
                need_rows = torch.where(live, 1, 2).to(torch.uint8).contiguous()
            else:
                need_rows = live.to(torch.uint8).contiguous()
        lse, logp, obar, flags = lm_head_forward(h2, w, tgt32, need, status, need_rows)
        if flags & nat.FLAG_TARGET_RANGE:
            L._raise_flags(nat.FLAG_TARGET_RANGE, check.kind)
        ctx.save_for_backward(h2, w, tgt32, lse, logp, obar)
        ctx.hidden_shape = hidden.shape
        ctx.set_materialize_grads(False)
        return logp.view(hidden.shape[:-1])

    @staticmethod
    def backward(ctx, g):
        need_h, need_w = ctx.needs_input_grad[1], ctx.needs_input_grad[2]
        if g is None or not (need_h or need_w):
            return None, None, None, None, None, None
        h2, w, tgt32, lse, logp, obar = ctx.saved_tensors
        gc = g.reshape(-1).to(torch.float32).contiguous()
        dh, dw = lm_head_backward(h2, w, tgt32, lse, logp, obar, gc, need_h, need_w)
        return (None, (dh.view(ctx.hidden_shape) if dh is not None else None), dw, None, None,
                None)


def linear_token_logprobs(hidden: Tensor, weight: Tensor, target_ids: Tensor, *,
                          row_block: int = DEFAULT_ROW_BLOCK) -> Tensor:
    """``gather_token_logprobs(hidden @ weight.T, target_ids)`` without the logits.

    ``hidden``: [..., H]; ``weight``: [V, H] (an LM head without bias, tied or
    not), both bfloat16, H a multiple of 128 up to 1024;
    ``target_ids``: hidden's prefix shape.  Returns float32 log-probs, as
    ``gather_token_logprobs`` does for 16-bit logits.  Differentiable into
    ``hidden`` and ``weight``.  ``row_block`` is accepted and unused: no more
    than a 32 x 64 logits tile exists at a time.
    """

    if row_block < 1:
        raise ValueError("row_block must be positive")
    return _cfg.as_reference_dtype(
        _LinearLogprobs.apply(L._params(nat.OBJ_PPO), hidden, weight, target_ids), hidden)


def linear_label_logprobs(hidden: Tensor, weight: Tensor, labels: Tensor,
                          ignore_index: int) -> Tensor:
    """:func:`linear_token_logprobs` for cross-entropy labels: a label equal to
    ``ignore_index`` has no target (log-prob 0, no gradient) and is exempt
    from the range check, whose failure raises IndexError as F.cross_entropy
    does."""

    p = nat.RrlPolicyParams()
    p.kind = nat.OBJ_NLL
    p.ignore_index = int(ignore_index)
    return _LinearLogprobs.apply(p, hidden, weight, labels, labels != int(ignore_index))


def fused_linear_policy_loss(
    hidden: Tensor,
    weight: Tensor,
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
    return_logprobs: bool = False,
    skip_masked_rows: bool = False,
    row_block: int = DEFAULT_ROW_BLOCK,
):
    """``fused_policy_loss(hidden @ weight.T, ...)`` without the logits tensor.

    ``hidden``: [..., H] final hidden states at the positions that predict
    ``target_ids`` (already shifted); ``weight``: the LM head's [V, H] weight
    (no bias).  Objectives and options as :func:`fused_policy_loss`; the loss
    is differentiable into ``hidden`` and ``weight``.  The log-probs come from
    the matrix-core LM head (:func:`linear_token_logprobs`) and feed the
    objective's kernels; its backward hands d loss / d logp back to the LM
    head's backward.  ``skip_masked_rows=True`` (a training step, with
    gradients asked for) leaves out every block of 64 consecutive tokens whose
    mask weights are all 0: their log-probs are taken as 0, which a masked
    token's term multiplies by 0, so the loss and the gradients are those of
    the full computation, without the log-sum-exp pass over those blocks (no
    reference counterpart).  ``row_block`` is accepted and unused.
    """

    if objective not in L._OBJECTIVES:
        raise ValueError(
            f"unknown objective {objective!r}; expected one of {sorted(L._OBJECTIVES)}")
    kind = L._OBJECTIVES[objective]
    _prepare(hidden, weight, target_ids)
    if skip_masked_rows and return_logprobs:
        raise ValueError("skip_masked_rows=True leaves masked log-probs uncomputed; "
                         "it cannot be combined with return_logprobs=True")
    if row_block < 1:
        raise ValueError("row_block must be positive")
    mask = L._on_device(action_mask, hidden)
    ppo = L._params(nat.OBJ_PPO)
    if kind in (nat.OBJ_GSPO, nat.OBJ_GSPO_TOKEN):
        logp = _LinearLogprobs.apply(ppo, hidden, weight, target_ids, mask,
                                     bool(skip_masked_rows))
        fn = L.gspo_policy_loss if kind == nat.OBJ_GSPO else L.gspo_token_policy_loss
        out = fn(logp, old_logprobs, advantages, action_mask, clip_low=clip_low,
                 clip_high=clip_low if clip_high is None else clip_high,
                 max_log_ratio=max_log_ratio)
        return (out, _cfg.as_reference_dtype(logp.detach(), hidden)) if return_logprobs else out

    p = L._token_local_params(kind, hidden.shape[:-1], old_logprobs, advantages, action_mask,
                              clip_low=clip_low, clip_high=clip_high,
                              max_log_ratio=max_log_ratio, detach_ratio=detach_ratio,
                              tau_positive=tau_positive, tau_negative=tau_negative)
    logp = _LinearLogprobs.apply(ppo, hidden, weight, target_ids, mask, bool(skip_masked_rows))
    obj, d1, d2, d3, _seq, trusted = L._objective(p, logp, old_logprobs, advantages, mask)
    out = L._token_local_output(kind, obj, d1, d2, d3, trusted)
    return (out, _cfg.as_reference_dtype(logp.detach(), hidden)) if return_logprobs else out
