"""Next-token cross-entropy (SFT loss) in one sweep per logits row.

The reference forms the language-model loss inside the model forwards
(rosetrainer/model.py:643-649, rosetrainer/qwen3.py:558-564)::

    shift_logits = logits[:, :-1, :].contiguous()
    shift_labels = labels[:, 1:].contiguous()
    loss = F.cross_entropy(shift_logits.view(-1, V), shift_labels.view(-1))

That copies the shifted logits, materialises a log-softmax over them, and its
backward writes a gradient for the shifted copy and then one for the full
logits.  Here the same loss is the objective kind NLL of the single-pass row
kernel (``rrl_fused_logprob_policy``): every logits row is read once, in place
through the shifted view, and its gradient row written once, with
d loss / d logp = -1/n for the n non-ignored tokens known before the sweep
(``rrl_policy_row_coef`` counts them).  The loss itself is the reduction of the
per-token log-probs (``rrl_policy_fwd``).

Semantics follow ``torch.nn.functional.cross_entropy`` with ``weight=None``
and ``label_smoothing=0`` (the reference's call): ``ignore_index`` tokens carry
no loss and are not range-checked; any other id outside ``[0, V)`` raises
``IndexError``; ``reduction="mean"`` over no tokens gives NaN and zero
gradients.  16-bit logits give a float32 loss (the reference returns the
logits dtype); arithmetic is float32 (float64 for float64 logits).
"""

from __future__ import annotations

from typing import Tuple

import torch
from torch import Tensor

from .. import _native as nat
from .. import _config as _cfg
from ..roserlhf import linear as _linear
from ..roserlhf import losses as _losses

__all__ = [
    "causal_lm_loss",
    "cross_entropy",
    "fused_linear_cross_entropy",
    "linear_causal_lm_loss",
]

_REDUCTIONS = ("mean", "sum")


def _nll_params(ignore_index: int, reduction: str) -> nat.RrlPolicyParams:
    if reduction not in _REDUCTIONS:
        if reduction == "none":
            raise ValueError("reduction='none' is not provided by the single-pass path; "
                             "use 'mean' or 'sum'")
        raise ValueError(f"{reduction} is not a valid value for reduction")
    p = nat.RrlPolicyParams()
    p.kind = nat.OBJ_NLL
    p.ignore_index = int(ignore_index)
    if reduction == "sum":
        p.flags |= nat.POLICY_SUM
    return p


def _check_labels(labels: Tensor) -> None:
    if labels.dtype not in (torch.int64, torch.int32):
        raise RuntimeError(f"expected scalar type Long but found {str(labels.dtype)[6:].capitalize()}")


def _unused_operand(dev: torch.device, acc: torch.dtype) -> Tuple[nat.RrlView, Tensor]:
    """The old-log-prob / advantage operands NLL does not read: one zero
    broadcast to every token."""

    z = torch.zeros(1, dtype=acc, device=dev)
    return nat.RrlView(z.data_ptr(), nat.dtype_code(acc), 0, 0), z


class _CrossEntropyRows(torch.autograd.Function):
    """-mean/sum of log_softmax(rows)[label] over non-ignored labels, with the
    gradient of every logits row written during the forward.

    ``shift=True`` takes logits [B, T, V] and labels [B, T] and scores rows
    (b, t < T-1) against labels (b, t+1) through strided views; the gradient
    rows of the last position are zero.  The forward leaves the gradient for
    an upstream d loss = 1; the backward rescales it on the device otherwise.
    """

    @staticmethod
    def forward(ctx, params: nat.RrlPolicyParams, inplace: bool, shift: bool, logits: Tensor,
                labels: Tensor):
        dev = nat.require_device(logits, labels)
        src, lab = (logits[:, :-1], labels[:, 1:]) if shift else (logits, labels)
        x, B, T, V, s_b, s_t = nat.logits_rows(src)
        if inplace and (x.data_ptr() != src.data_ptr() or logits.stride(-1) != 1):
            raise RuntimeError("inplace=True needs logits whose rows can be addressed in place")
        tview, tkeep = nat.rows_view(lab, B, T)
        acc = nat.acc_dtype(logits.dtype)
        acc_code = nat.dtype_code(acc)
        stream = nat.stream_ptr(dev)
        unused, keep0 = _unused_operand(dev, acc)
        ws = torch.empty(nat.lib().rrl_policy_workspace_bytes(B, acc_code), dtype=torch.uint8,
                         device=dev)
        coef = torch.empty(B, dtype=acc, device=dev)
        records = torch.empty(nat.lib().rrl_fused_records_bytes(B, T), dtype=torch.uint8,
                              device=dev)
        logp = torch.empty(B * T, dtype=acc, device=dev)
        lse = torch.empty(B * T, dtype=acc, device=dev)
        scal = torch.empty(nat.NSCALARS, dtype=acc, device=dev)
        if inplace:
            dl = logits
            d_b, d_t = s_b, s_t
            dptr = x.data_ptr()
        else:
            dl = torch.empty(logits.shape, dtype=logits.dtype, device=dev)
            if shift:
                d_b, d_t = dl.stride(0), dl.stride(1)
            else:
                d_b, d_t = T * V, V
            dptr = dl.data_ptr()
        lview = nat.RrlView(logp.data_ptr(), acc_code, T, 1)

        early = _losses._check_before_sweep(logits, inplace)
        rerun = _losses._rerun_on_device(logits, inplace)

        def run(p):
            status = nat.new_status(dev)
            pref = _losses.ctypes_ref(p)
            nat.call("rrl_policy_row_coef", pref, B, T, tview, acc_code, coef.data_ptr(),
                     ws.data_ptr(), status.data_ptr(), stream)
            if early:
                nat.call("rrl_check_targets", pref, B, T, V, tview, status.data_ptr(), stream)
                _losses._raise_flags(nat.read_status(status), nat.OBJ_NLL)
            for q in (pref, _losses.ctypes_ref(_losses._rerun_params(p))) if rerun else (pref,):
                nat.call("rrl_fused_logprob_policy", q, x.data_ptr(), nat.dtype_code(x.dtype), B,
                         T, V, s_b, s_t, tview, unused, unused, tview, coef.data_ptr(),
                         records.data_ptr(), logp.data_ptr(), lse.data_ptr(), dptr,
                         nat.dtype_code(logits.dtype), d_b, d_t, status.data_ptr(), stream,
                         timed=q is pref)
            nat.call("rrl_policy_fwd", pref, B, T, lview, unused, unused, tview, acc_code,
                     ws.data_ptr(), scal.data_ptr(), None, None, status.data_ptr(), stream)
            return 0 if early else nat.read_status(status)

        flags = run(params)
        if flags & nat.FLAG_FAST_RANGE:
            # A row's log-sum-exp lies beyond the register-resident 16-bit kernel's exponent
            # range: redo the call on the generic row kernel.
            if inplace:
                raise RuntimeError(
                    "cross-entropy with inplace=True: logits beyond +-2e38 need the generic "
                    "kernel, which cannot rerun over overwritten logits; call with inplace=False")
            generic = nat.RrlPolicyParams.from_buffer_copy(params)
            generic.flags |= nat.POLICY_GENERIC
            flags = run(generic)
        _losses._raise_flags(flags, nat.OBJ_NLL)
        if shift and logits.shape[1] > 0:
            dl[:, -1].zero_()  # the last position predicts nothing
        del keep0, tkeep
        # Row geometry of the whole gradient tensor for the backward's rescale:
        # in place it is the caller's logits, which may be a strided view (a
        # padded-vocabulary slice, a [:, :-1] shift) whose rows are not V apart.
        gx, gB, gT, gV, gs_b, gs_t = nat.logits_rows(dl)
        if gx.data_ptr() != dl.data_ptr():
            raise RuntimeError("cross-entropy gradient rows cannot be addressed in place")
        ctx.dl = dl
        ctx.geom = (gB, gT, gV, gs_b, gs_t)
        ctx.set_materialize_grads(False)
        return -scal[0]

    @staticmethod
    def backward(ctx, g):
        dl = ctx.dl
        ctx.dl = None
        if g is None or dl is None or not ctx.needs_input_grad[3]:
            return None, None, None, None, None
        B, T, V, s_b, s_t = ctx.geom
        scale = g.reshape(1).to(torch.float64 if dl.dtype == torch.float64 else torch.float32)
        nat.call("rrl_scale_rows", dl.data_ptr(), nat.dtype_code(dl.dtype), B, T, V, s_b, s_t,
                 scale.data_ptr(), nat.dtype_code(scale.dtype), 1.0, nat.stream_ptr(dl.device))
        return None, None, None, dl, None


def cross_entropy(input: Tensor, target: Tensor, *, ignore_index: int = -100,
                  reduction: str = "mean", inplace: bool = False) -> Tensor:
    """``F.cross_entropy(input, target, ignore_index=..., reduction=...)`` with
    the class dimension last: ``input`` [..., V] logits, ``target`` integer ids
    of ``input.shape[:-1]`` (the reference calls it on ``[N, V]`` and ``[N]``,
    rosetrainer/model.py:645-648).

    One read of each logits row and one write of its gradient row.
    ``inplace=True`` writes the gradient over ``input`` (the logits are
    destroyed; backward may then run once).
    """

    if input.ndim < 2:
        raise ValueError("input must be [..., C] logits with the class dimension last")
    _check_labels(target)
    if tuple(input.shape[:-1]) != tuple(target.shape):
        n_in = input.numel() // max(int(input.shape[-1]), 1) if input.shape[-1] else 0
        raise ValueError(
            f"Expected input batch_size ({n_in}) to match target batch_size ({target.numel()}).")
    p = _nll_params(ignore_index, reduction)
    return _cfg.as_reference_dtype(
        _CrossEntropyRows.apply(p, bool(inplace), False, input, target), input)


def causal_lm_loss(logits: Tensor, labels: Tensor, *, ignore_index: int = -100,
                   reduction: str = "mean", inplace: bool = False) -> Tensor:
    """The reference's LM loss, rosetrainer/model.py:643-649 (and
    qwen3.py:558-564): position t's logits score label t+1.

    ``logits`` [B, T, V], ``labels`` [B, T].  No shifted copy is made; the
    returned gradient has the logits' shape with zero rows at t = T-1.
    """

    if logits.ndim != 3:
        raise ValueError("logits must be [batch, positions, vocabulary]")
    _check_labels(labels)
    if tuple(labels.shape) != tuple(logits.shape[:2]):
        raise ValueError(
            f"labels shape {tuple(labels.shape)} must match logits prefix {tuple(logits.shape[:2])}")
    p = _nll_params(ignore_index, reduction)
    return _cfg.as_reference_dtype(
        _CrossEntropyRows.apply(p, bool(inplace), True, logits, labels), logits)


def fused_linear_cross_entropy(hidden: Tensor, weight: Tensor, target: Tensor, *,
                               ignore_index: int = -100, reduction: str = "mean",
                               row_block: int = _linear.DEFAULT_ROW_BLOCK,
                               impl: str = "auto") -> Tensor:
    """``cross_entropy(hidden @ weight.T, target)`` without the whole logits
    tensor.

    ``hidden`` [..., H] (positions already aligned with ``target``),
    ``weight`` the LM head's [V, H] (no bias: rosetrainer/model.py:499,
    qwen3.py:508), one float dtype.  The label log-probs come from the LM head
    (``linear_label_logprobs``: ignored labels have no target and are never
    computed), the loss from the NLL objective's kernels.  ``impl``: as
    ``fused_linear_policy_loss`` (``"chunked"``: row blocks of at most
    ``row_block`` tokens of logits, any float dtype and hidden size;
    ``"tiles"``: the hand-written MFMA kernels, bfloat16 with a hidden size
    that is a multiple of 128 up to 1024).
    """

    _linear._prepare(hidden, weight, target)
    _check_labels(target)
    p = _nll_params(ignore_index, reduction)
    if row_block < 1:
        raise ValueError("row_block must be positive")
    dev = nat.require_device(hidden, weight, target)
    logp = _linear.linear_label_logprobs(hidden, weight, target, ignore_index,
                                         row_block=row_block, impl=impl)
    unused = torch.zeros((), dtype=torch.float32, device=dev).expand(target.shape)
    obj = _losses._objective(p, logp, unused, unused, target)[0]
    return _cfg.as_reference_dtype(-obj, hidden)


def linear_causal_lm_loss(hidden: Tensor, weight: Tensor, labels: Tensor, *,
                          ignore_index: int = -100, reduction: str = "mean",
                          row_block: int = _linear.DEFAULT_ROW_BLOCK,
                          impl: str = "auto") -> Tensor:
    """rosetrainer/model.py:641-649 from the final hidden states: the LM head,
    the causal shift and the cross-entropy, without the logits tensor.
    ``hidden`` [B, T, H], ``labels`` [B, T]."""

    if hidden.ndim != 3:
        raise ValueError("hidden must be [batch, positions, hidden]")
    if tuple(labels.shape) != tuple(hidden.shape[:2]):
        raise ValueError(
            f"labels shape {tuple(labels.shape)} must match hidden prefix {tuple(hidden.shape[:2])}")
    return fused_linear_cross_entropy(hidden[:, :-1], weight, labels[:, 1:],
                                      ignore_index=ignore_index, reduction=reduction,
                                      row_block=row_block, impl=impl)
