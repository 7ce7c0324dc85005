"""Fused LM-head + token log-prob + policy objective, without the logits tensor.

The neighbour of the hot path on the producer side: the reference forms
``logits = lm_head(hidden)`` (``rosetrainer/model.py:499,641``,
``rosetrainer/qwen3.py:508,556``, no bias) and then calls
``gather_token_logprobs`` (``roserlhf/losses.py:14-38``) and an objective,
holding the whole ``[tokens, V]`` logits tensor (79.7 GB at 262,144 tokens x
151,936 vocab in bf16) plus its gradient.

Here the tokens are cut into row blocks (whole sequences, or stretches of one
long sequence).  For each block:

1. ``logits_blk = hidden_blk @ weight.T`` into one reused HBM buffer
   (hipBLASLt GEMM on the MFMA units);
2. for the token-local objectives (PPO/GRPO clip, SAO, SAPO) the single-pass
   row kernel of ``fused_policy_loss`` reads the block once and writes
   ``dlogits_blk`` over it (the mask denominators, known from the masks alone,
   come first from ``rrl_policy_row_coef`` over the whole batch);
3. ``dhidden_blk = dlogits_blk @ weight`` and ``dW += dlogits_blk.T @ hidden_blk``
   (float32 accumulation across blocks).

That is the three GEMMs of the composed step, 3 x 2·N·H·V flops, with no
recomputation, and the logits never exist beyond one block.  GSPO needs every
token's log-prob before any gradient: its forward sweeps the blocks for
log-probs only (``rrl_logprob_fwd``) and its backward sweeps them again,
recomputing each block's logits (4 x 2·N·H·V).
"""

from __future__ import annotations

from typing import List, Optional, Tuple

import torch
from torch import Tensor

from .. import _native as nat
from . import losses as L

__all__ = ["fused_linear_policy_loss", "linear_token_logprobs"]

DEFAULT_ROW_BLOCK = 16384

# How dW accumulates across row blocks; resolved on first use per process
# (the float32-output GEMM overloads of torch.addmm/torch.mm run on ROCm).
_DW_MODE: Optional[str] = None


def _dw_mode(dev: torch.device) -> str:
    """"addmm" (bf16 x bf16 GEMM accumulating into float32 through
    torch.addmm's out_dtype form), "mm" (float32-output GEMM plus an add) or
    "cast" (16-bit GEMM output widened, then added)."""

    global _DW_MODE
    if _DW_MODE is None:
        a = torch.ones(2, 3, dtype=torch.bfloat16, device=dev)
        b = torch.ones(2, 4, dtype=torch.bfloat16, device=dev)
        acc = torch.ones(3, 4, dtype=torch.float32, device=dev)
        try:
            torch.addmm(acc, a.t(), b, out_dtype=torch.float32, out=acc)
            ok = bool((acc == 3).all())
            _DW_MODE = "addmm" if ok else None
        except (RuntimeError, TypeError):
            _DW_MODE = None
        if _DW_MODE is None:
            try:
                r = torch.mm(a.t(), b, out_dtype=torch.float32)
                _DW_MODE = "mm" if r.dtype == torch.float32 and bool((r == 2).all()) else "cast"
            except (RuntimeError, TypeError):
                _DW_MODE = "cast"
    return _DW_MODE


class _Blocks:
    """Row blocks of a [B, T] token grid and the GEMMs around each block.

    A block is whole sequences ``b0:b1`` when a sequence has at most
    ``row_block`` tokens, else a stretch ``t0:t1`` of one sequence; either way
    its tokens are contiguous rows ``r0 : r0 + rows`` of ``hidden.view(B*T, H)``.
    """

    def __init__(self, hidden2: Tensor, weight: Tensor, B: int, T: int, row_block: int):
        if row_block < 1:
            raise ValueError("row_block must be positive")
        self.h, self.w = hidden2, weight
        self.B, self.T = B, T
        self.V, self.H = weight.shape
        blocks: List[Tuple[int, int, int, int]] = []
        if T <= row_block:
            bc = max(1, row_block // max(T, 1))
            blocks = [(b0, min(B, b0 + bc), 0, T) for b0 in range(0, B, bc)]
        else:
            blocks = [(b, b + 1, t0, min(T, t0 + row_block))
                      for b in range(B) for t0 in range(0, T, row_block)]
        self.blocks = blocks
        rows = max((b1 - b0) * (t1 - t0) for b0, b1, t0, t1 in blocks) if blocks else 0
        self.buf = torch.empty((rows, self.V), dtype=hidden2.dtype, device=hidden2.device)

    @staticmethod
    def rows(blk) -> int:
        b0, b1, t0, t1 = blk
        return (b1 - b0) * (t1 - t0)

    def r0(self, blk) -> int:
        return blk[0] * self.T + blk[2]

    def logits(self, blk) -> Tensor:
        n = self.rows(blk)
        r0 = self.r0(blk)
        x = self.buf[:n]
        torch.mm(self.h[r0:r0 + n], self.w.t(), out=x)
        return x

    def grads(self, blk, d: Tensor, dh: Optional[Tensor], dw: Optional[Tensor],
              first: bool) -> None:
        """dhidden rows of the block, and the block's share of dW: written when
        dW is in the weight dtype (one block), accumulated when float32."""

        n = self.rows(blk)
        r0 = self.r0(blk)
        h = self.h[r0:r0 + n]
        if dh is not None:
            torch.mm(d, self.w, out=dh[r0:r0 + n])
        if dw is None:
            return
        if dw.dtype == d.dtype:
            if first:
                torch.mm(d.t(), h, out=dw)
            else:
                torch.addmm(dw, d.t(), h, out=dw)
            return
        # 16-bit dlogits into the float32 accumulator
        mode = _dw_mode(d.device)
        if mode == "addmm":
            torch.addmm(dw, d.t(), h, beta=0.0 if first else 1.0, out_dtype=torch.float32,
                        out=dw)
            return
        if mode == "mm":
            part = torch.mm(d.t(), h, out_dtype=torch.float32)
        else:
            part = torch.mm(d.t(), h).to(torch.float32)
        if first:
            dw.copy_(part)
        else:
            dw.add_(part)

    def views(self, blk, *ts: Tensor):
        """[rows, cols] views of [B, T] operands restricted to the block."""

        b0, b1, t0, t1 = blk
        out = []
        for t in ts:
            v, keep = nat.rows_view(t[b0:b1, t0:t1], b1 - b0, t1 - t0)
            out.append((v, keep))
        return out


def _grad_buffers(blocks: _Blocks, hidden2: Tensor, weight: Tensor, need_h: bool,
                  need_w: bool):
    dh = torch.empty_like(hidden2) if need_h else None
    dw = None
    if need_w:
        wide = len(blocks.blocks) > 1 and weight.dtype in (torch.bfloat16, torch.float16)
        dw = torch.empty(weight.shape, dtype=torch.float32 if wide else weight.dtype,
                         device=weight.device)
        if sum(blocks.rows(b) for b in blocks.blocks) == 0:
            dw.zero_()
    return dh, dw


def _backward_sweep(blocks: _Blocks, tgt: Tensor, lse: Tensor, logp: Tensor, g: Tensor,
                    need_h: bool, need_w: bool, stream: int):
    """dhidden, dW for d loss / d logp = g: each block's logits are recomputed,
    turned into dlogits in place by rrl_logprob_bwd, then fed to the GEMMs."""

    dh, dw = _grad_buffers(blocks, blocks.h, blocks.w, need_h, need_w)
    V = blocks.V
    dt = nat.dtype_code(blocks.h.dtype)
    done = 0
    for blk in blocks.blocks:
        n = blocks.rows(blk)
        if n == 0:
            continue
        r0 = blocks.r0(blk)
        bc, tc = blk[1] - blk[0], blk[3] - blk[2]
        x = blocks.logits(blk)
        (tv, _tk), = blocks.views(blk, tgt)
        nat.call("rrl_logprob_bwd", x.data_ptr(), dt, bc, tc, V, tc * V, V, tv,
                 lse[r0:].data_ptr(), logp[r0:].data_ptr(), g[r0:].data_ptr(), x.data_ptr(), dt,
                 tc * V, V, 0, stream)
        blocks.grads(blk, x, dh, dw, first=(done == 0))
        done += 1
    return dh, dw


def _finish_grads(dh, dw, hidden_shape, weight_dtype: torch.dtype):
    gh = dh.view(hidden_shape) if dh is not None else None
    gw = None
    if dw is not None:
        gw = dw if dw.dtype == weight_dtype else dw.to(weight_dtype)
    return gh, gw


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


class _LinearLogprobs(torch.autograd.Function):
    """log_softmax(hidden @ weight.T)[target], one row block of logits at a time;
    the backward recomputes each block's logits."""

    @staticmethod
    def forward(ctx, row_block: int, hidden: Tensor, weight: Tensor, target_ids: Tensor):
        dev = nat.require_device(hidden, weight, target_ids)
        B, T = _prepare(hidden, weight, target_ids)
        H = hidden.shape[-1]
        h2 = hidden.reshape(B * T, H).contiguous()
        w = weight.contiguous()
        blocks = _Blocks(h2, w, B, T, row_block)
        tgt = target_ids.reshape(B, T)
        acc = nat.acc_dtype(hidden.dtype)
        acc_code = nat.dtype_code(acc)
        logp = torch.empty(B * T, dtype=acc, device=dev)
        lse = torch.empty(B * T, dtype=acc, device=dev)
        status = nat.new_status(dev)
        stream = nat.stream_ptr(dev)
        V = blocks.V
        dt = nat.dtype_code(hidden.dtype)
        for blk in blocks.blocks:
            n = blocks.rows(blk)
            if n == 0:
                continue
            r0 = blocks.r0(blk)
            bc, tc = blk[1] - blk[0], blk[3] - blk[2]
            x = blocks.logits(blk)
            (tv, _tk), = blocks.views(blk, tgt)
            nat.call("rrl_logprob_fwd", x.data_ptr(), dt, bc, tc, V, tc * V, V, tv,
                     logp[r0:].data_ptr(), acc_code, lse[r0:].data_ptr(), status.data_ptr(),
                     stream)
        blocks.buf = None
        if nat.read_status(status) & nat.FLAG_TARGET_RANGE:
            L._raise_target_range()
        ctx.row_block = row_block
        ctx.save_for_backward(h2, w, tgt, lse, logp)
        ctx.shapes = (hidden.shape, B, T)
        return logp.view(hidden.shape[:-1])

    @staticmethod
    def backward(ctx, g):
        need_h, need_w = ctx.needs_input_grad[1], ctx.needs_input_grad[2]
        if g is None or not (need_h or need_w):
            return None, None, None, None
        h2, w, tgt, lse, logp = ctx.saved_tensors
        shape, B, T = ctx.shapes
        gc = g.reshape(B * T).to(lse.dtype).contiguous()
        blocks = _Blocks(h2, w, B, T, ctx.row_block)
        dh, dw = _backward_sweep(blocks, tgt, lse, logp, gc, need_h, need_w,
                                 nat.stream_ptr(lse.device))
        gh, gw = _finish_grads(dh, dw, shape, w.dtype)
        return None, gh, gw, None


def linear_token_logprobs(hidden: Tensor, weight: Tensor, target_ids: Tensor, *,
                          row_block: int = DEFAULT_ROW_BLOCK) -> Tensor:
    """``gather_token_logprobs(hidden @ weight.T, target_ids)`` without the logits.

    ``hidden``: [..., H]; ``weight``: [V, H] (an LM head without bias, tied or
    not); ``target_ids``: hidden's prefix shape.  16-bit inputs give float32
    log-probs, as ``gather_token_logprobs`` does for 16-bit logits.  The logits
    exist only ``row_block`` tokens at a time; the backward recomputes them.
    """

    return _LinearLogprobs.apply(int(row_block), hidden, weight, target_ids)


class _FusedLinearPolicy(torch.autograd.Function):
    """Token-local objective over ``hidden @ weight.T`` in one sweep of row blocks.

    The forward leaves dhidden and dW for an upstream d loss = 1; backward
    rescales them on the device for another scale and, when diagnostics also
    receive gradients, recomputes through the backward sweep.
    """

    @staticmethod
    def forward(ctx, params: nat.RrlPolicyParams, row_block: int, hidden: Tensor,
                weight: Tensor, target_ids: Tensor, old: Tensor, adv: Tensor, mask: Tensor):
        kind = params.kind
        dev = nat.require_device(hidden, weight, target_ids, old, adv, mask)
        B, T = _prepare(hidden, weight, target_ids)
        H = hidden.shape[-1]
        h2 = hidden.reshape(B * T, H).contiguous()
        w = weight.contiguous()
        blocks = _Blocks(h2, w, B, T, row_block)
        V = blocks.V
        tgt, old2, adv2, mask2 = (t.reshape(B, T) for t in (target_ids, old, adv, mask))
        acc = nat.acc_dtype(hidden.dtype)
        acc_code = nat.dtype_code(acc)
        dt = nat.dtype_code(hidden.dtype)
        stream = nat.stream_ptr(dev)
        need_h, need_w = ctx.needs_input_grad[2], ctx.needs_input_grad[3]
        ws = torch.empty(nat.lib().rrl_policy_workspace_bytes(B, acc_code), dtype=torch.uint8,
                         device=dev)
        coef = torch.empty(B, dtype=acc, device=dev)
        max_bc = max((b[1] - b[0] for b in blocks.blocks), default=0)
        max_tc = max((b[3] - b[2] for b in blocks.blocks), default=0)
        records = torch.empty(nat.lib().rrl_fused_records_bytes(max_bc, max_tc),
                              dtype=torch.uint8, device=dev)
        logp = torch.empty(B * T, dtype=acc, device=dev)
        lse = torch.empty(B * T, dtype=acc, device=dev)
        scal = torch.empty(nat.NSCALARS, dtype=acc, device=dev)
        trusted = torch.empty(B * T if kind == nat.OBJ_SAO else 0, dtype=torch.bool, device=dev)
        mv_full, _mk = nat.rows_view(mask2, B, T)
        ov_full, _ok = nat.rows_view(old2, B, T)
        av_full, _ak = nat.rows_view(adv2, B, T)
        lview = nat.RrlView(logp.data_ptr(), acc_code, T, 1)

        def sweep(p):
            status = nat.new_status(dev)
            pref = L.ctypes_ref(p)
            dh, dw = _grad_buffers(blocks, h2, w, need_h, need_w)
            nat.call("rrl_policy_row_coef", pref, B, T, mv_full, acc_code, coef.data_ptr(),
                     ws.data_ptr(), status.data_ptr(), stream)
            done = 0
            for blk in blocks.blocks:
                n = blocks.rows(blk)
                if n == 0:
                    continue
                r0 = blocks.r0(blk)
                bc, tc = blk[1] - blk[0], blk[3] - blk[2]
                x = blocks.logits(blk)
                (tv, _a), (ov, _b), (av, _c), (mv, _d) = blocks.views(blk, tgt, old2, adv2, mask2)
                nat.call("rrl_fused_logprob_policy", pref, x.data_ptr(), dt, bc, tc, V, tc * V,
                         V, tv, ov, av, mv, coef[blk[0]:].data_ptr(), records.data_ptr(),
                         logp[r0:].data_ptr(), lse[r0:].data_ptr(), x.data_ptr(), dt, tc * V, V,
                         status.data_ptr(), stream)
                blocks.grads(blk, x, dh, dw, first=(done == 0))
                done += 1
            nat.call("rrl_policy_fwd", pref, B, T, lview, ov_full, av_full, mv_full, acc_code,
                     ws.data_ptr(), scal.data_ptr(), None,
                     nat.ptr(trusted) if trusted.numel() else None, status.data_ptr(), stream)
            return nat.read_status(status), dh, dw

        flags, dh, dw = sweep(params)
        if flags & nat.FLAG_FAST_RANGE:
            # Some row's log-sum-exp lies beyond the register-resident 16-bit kernel's
            # exponent range: the logits are recomputed anyway, so redo the
            # sweep on the generic row kernel.
            generic = nat.RrlPolicyParams.from_buffer_copy(params)
            generic.flags |= nat.POLICY_GENERIC
            flags, dh, dw = sweep(generic)
        blocks.buf = None
        L._raise_flags(flags, kind)
        gh, gw = _finish_grads(dh, dw, hidden.shape, w.dtype)

        ctx.params = params
        ctx.row_block = row_block
        ctx.pre = (gh, gw)
        ctx.shapes = (hidden.shape, B, T, acc)
        ctx.save_for_backward(h2, w, tgt, old2, adv2, mask2, lse, logp, ws)
        ctx.set_materialize_grads(False)
        dts = L._scalar_dtypes(kind, logp, old, adv)
        outs = [scal[k].to(dts[k], copy=True) for k in range(4)]
        logp_out = logp.view(hidden.shape[:-1])
        trusted_out = trusted.view(hidden.shape[:-1]) if kind == nat.OBJ_SAO else trusted
        if kind in (nat.OBJ_PPO, nat.OBJ_SAO):
            ctx.mark_non_differentiable(outs[2], logp_out, trusted_out)
        else:
            ctx.mark_non_differentiable(logp_out, trusted_out)
        return outs[0], outs[1], outs[2], outs[3], logp_out, trusted_out

    @staticmethod
    def backward(ctx, g0, g1, g2, g3, _glogp, _gtrusted):
        need_h, need_w = ctx.needs_input_grad[2], ctx.needs_input_grad[3]
        if not (need_h or need_w):
            return (None,) * 8
        params = ctx.params
        shape, B, T, acc = ctx.shapes
        h2, w, tgt, old2, adv2, mask2, lse, logp, ws = ctx.saved_tensors
        dev = lse.device
        stream = nat.stream_ptr(dev)
        gh, gw = ctx.pre if ctx.pre is not None else (None, None)
        ctx.pre = None
        extra = any(g is not None for g in (g1, g3)) or (
            params.kind == nat.OBJ_SAPO and g2 is not None)
        if (gh is not None or gw is not None) and not extra:
            scale = (-g0).reshape(1).to(acc) if g0 is not None else torch.zeros(
                1, dtype=acc, device=dev)
            for t in (gh, gw):
                if t is not None:
                    n, c = t.numel() // t.shape[-1], t.shape[-1]
                    nat.call("rrl_scale_rows", t.data_ptr(), nat.dtype_code(t.dtype), 1, n, c,
                             0, c, scale.data_ptr(), nat.dtype_code(acc), 1.0, stream)
            return (None, None, gh, gw, None, None, None, None)
        # Diagnostics receive gradients too: full d/d logp, then the
        # recomputing backward sweep.
        gs = torch.zeros(nat.NSCALARS, dtype=acc, device=dev)
        for k, g in enumerate((g0, g1, g2, g3)):
            if g is not None:
                gs[k] = g.to(acc)
        acc_code = nat.dtype_code(acc)
        lview = nat.RrlView(logp.data_ptr(), acc_code, T, 1)
        ov, _a = nat.rows_view(old2, B, T)
        av, _b = nat.rows_view(adv2, B, T)
        mv, _c = nat.rows_view(mask2, B, T)
        gcur = torch.empty(B * T, dtype=acc, device=dev)
        nat.call("rrl_policy_bwd", L.ctypes_ref(params), B, T, lview, ov, av, mv, acc_code,
                 ws.data_ptr(), gs.data_ptr(), None, gcur.data_ptr(), stream)
        blocks = _Blocks(h2, w, B, T, ctx.row_block)
        dh, dw = _backward_sweep(blocks, tgt, lse, logp, gcur, need_h, need_w, stream)
        gh, gw = _finish_grads(dh, dw, shape, w.dtype)
        return (None, None, gh, gw, None, None, None, None)


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
    is differentiable into ``hidden`` and ``weight``.  The token-local
    objectives compute dhidden and dW during the forward (three GEMMs per row
    block, no recomputation); GSPO's forward keeps only log-probs and its
    backward recomputes the logits.  ``row_block`` tokens of logits (plus
    their in-place gradient) exist at a time: 16,384 x 151,936 bf16 is 5 GB.
    """

    if objective not in L._OBJECTIVES:
        raise ValueError(
            f"unknown objective {objective!r}; expected one of {sorted(L._OBJECTIVES)}")
    kind = L._OBJECTIVES[objective]
    _prepare(hidden, weight, target_ids)
    if skip_masked_rows and return_logprobs:
        raise ValueError("skip_masked_rows=True leaves masked log-probs uncomputed; "
                         "it cannot be combined with return_logprobs=True")
    if kind in (nat.OBJ_GSPO, nat.OBJ_GSPO_TOKEN):
        if skip_masked_rows:
            raise ValueError("skip_masked_rows=True applies to the single-sweep objectives only")
        logp = linear_token_logprobs(hidden, weight, target_ids, row_block=row_block)
        fn = L.gspo_policy_loss if kind == nat.OBJ_GSPO else L.gspo_token_policy_loss
        out = fn(logp, old_logprobs, advantages, action_mask, clip_low=clip_low,
                 clip_high=clip_low if clip_high is None else clip_high,
                 max_log_ratio=max_log_ratio)
        return (out, logp.detach()) if return_logprobs else out

    p = L._token_local_params(kind, hidden.shape[:-1], old_logprobs, advantages, action_mask,
                              clip_low=clip_low, clip_high=clip_high,
                              max_log_ratio=max_log_ratio, detach_ratio=detach_ratio,
                              tau_positive=tau_positive, tau_negative=tau_negative)
    if skip_masked_rows:
        p.flags |= nat.POLICY_SKIP_MASKED
    mask = L._on_device(action_mask, hidden)
    obj, d1, d2, d3, logp, trusted = _FusedLinearPolicy.apply(
        p, int(row_block), hidden, weight, target_ids, old_logprobs, advantages, mask)
    out = L._token_local_output(kind, obj, d1, d2, d3, trusted)
    return (out, logp) if return_logprobs else out
