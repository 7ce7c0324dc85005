"""Fused LM-head + token log-prob + policy objective (config 5).

The neighbour of the hot path on the producer side: the reference forms
``logits = lm_head(hidden)`` (``rosetrainer/model.py:499,641``,
``rosetrainer/qwen3.py:508,556``, no bias) and then calls
``gather_token_logprobs`` (``roserlhf/losses.py:14-38``) and an objective,
holding the whole ``[tokens, V]`` logits tensor (79.7 GB at 262,144 tokens x
151,936 vocab in bf16) plus its gradient.

Two implementations sit behind one API (``impl``):

* ``"chunked"`` (what ``"auto"`` selects): the tokens go through in row
  blocks of at most ``row_block`` tokens, the logits of one block at a time
  in one reused buffer.  The three products are plain GEMMs (the GEMM library
  through ``torch.mm``); the work between them is this package's row kernels
  on the block: log-sum-exp and log-probs, the objective's d loss / d logp
  and dlogits written over the block's logits.  Only tokens whose
  d loss / d logp can be non-zero (mask weight != 0) go through the gradient
  products; the others take a log-sum-exp pass alone.  Every logit is the
  GEMM's, rounded to the weight dtype as the reference's ``F.linear`` leaves
  it.  For the token-local objectives (PPO/GRPO clip, SAO, SAPO) one sweep
  of each block of active tokens does everything, so every logit is formed
  once; GSPO's sequence ratio needs every log-prob before any gradient, and
  its backward forms the active blocks' logits a second time.  Any float
  dtype, any hidden size.
* ``"tiles"``: hand-written gfx950 MFMA kernels (``csrc/lm_head.hip``) that
  never hold more than a 32 x 64 logits tile.  The forward streams the
  vocabulary past 64-token blocks with an online softmax per token and forms
  ``obar_n = sum_{v != a_n} p_nv W_v`` in the same pass; ``dhidden_n =
  g_n ((1 - p_target) W[a_n] - obar_n)`` is an elementwise kernel; ``dW``
  streams the tokens past 64-row blocks of the weight, recomputing each
  logits tile from the saved log-sum-exp.  bfloat16, hidden sizes that are
  multiples of 128 up to 1024.  4 x 2·N·H·V flops for an all-active batch.

Both compose with any objective of the package through autograd: the
log-probs are an ordinary differentiable tensor.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from .. import _native as nat
from .. import _config as _cfg
from . import losses as L

__all__ = ["fused_linear_policy_loss", "linear_token_logprobs"]

# Tokens per row block of the chunked path (5 GB of bf16 logits at V = 151,936).
DEFAULT_ROW_BLOCK = 16384
IMPLS = ("auto", "chunked", "tiles")

# The tile path's softmax weights pass through the MFMA as 16-bit values:
# bfloat16 holds weights of order 1/V; float16's normal range stops at 6.1e-5.
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


def _resolve_impl(impl: str, hidden: Tensor) -> str:
    if impl not in IMPLS:
        raise ValueError(f"unknown impl {impl!r}; expected one of {IMPLS}")
    if impl == "tiles":
        _check_mfma(hidden)
        return "tiles"
    return "chunked"


def _check_row_block(row_block: int) -> None:
    if row_block < 1:
        raise ValueError("row_block must be positive")


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


# ---------------------------------------------------------------------------
# Chunked path: library GEMMs per row block + the package's row kernels
# ---------------------------------------------------------------------------


_TAP: Optional[list] = None


class record_logits:
    """Testing aid for the chunked path: while active, every row block's
    logits (the GEMM's output, before the row kernels write over them) are
    kept in ``blocks`` as (token rows, logits) pairs, so that a check can run
    its oracle on exactly the logits the path consumed."""

    def __enter__(self):
        global _TAP
        self.blocks = []
        _TAP = self.blocks
        return self

    def __exit__(self, *exc):
        global _TAP
        _TAP = None
        return False


class _Blocks:
    """Row blocks of at most ``row_block`` tokens and one reused logits
    buffer ([row_block, V] in the weight dtype)."""

    def __init__(self, w: Tensor, row_block: int, n_rows: int):
        self.w = w
        self.V = w.shape[0]
        self.cap = max(1, min(int(row_block), int(n_rows)))
        self._buf: Optional[Tensor] = None

    def spans(self, n: int):
        return ((c0, min(n, c0 + self.cap)) for c0 in range(0, n, self.cap))

    def logits(self, x: Tensor, rows: Tensor) -> Tensor:
        """x [n, H], the hidden states of token rows ``rows`` -> the block's
        logits x @ W^T, [n, V] (the buffer's rows)."""

        n = x.shape[0]
        if self._buf is None:
            self._buf = torch.empty((self.cap, self.V), dtype=self.w.dtype, device=self.w.device)
        out = self._buf[:n]
        with nat.timed("lm_logits_gemm"):
            torch.mm(x, self.w.t(), out=out)
        if _TAP is not None:
            _TAP.append((rows.clone(), out.clone()))
        return out


_ADDMM_OUT_DTYPE: Optional[bool] = None


def _addmm_into(acc: Tensor, a: Tensor, b: Tensor) -> None:
    """acc += a @ b, with 16-bit a, b accumulated into a float32 acc."""

    global _ADDMM_OUT_DTYPE
    if acc.dtype == a.dtype:
        torch.addmm(acc, a, b, out=acc)
        return
    if _ADDMM_OUT_DTYPE is not False:
        try:
            torch.addmm(acc, a, b, out_dtype=acc.dtype, out=acc)
            _ADDMM_OUT_DTYPE = True
            return
        except (RuntimeError, TypeError):
            _ADDMM_OUT_DTYPE = False
    acc.add_(torch.mm(a, b).to(acc.dtype))


def _transposed16(w: Tensor) -> Tensor:
    """A contiguous [H, V] copy of a 2-byte [V, H] matrix (rrl_transpose16)."""

    V, H = w.shape
    out = torch.empty((H, V), dtype=w.dtype, device=w.device)
    nat.call("rrl_transpose16", w.data_ptr(), V, H, w.stride(0), out.data_ptr(), V,
             nat.stream_ptr(w.device))
    return out


class _Grads:
    """d hidden rows and the d weight accumulator of one chunked backward.

    For 16-bit weights both products take the operand layouts the GEMM library
    runs fastest on this GPU (measured on config 5's 16,384-token blocks):
    d hidden as ``dl @ wT.t()`` with ``wT`` a contiguous [H, V] copy of the
    weight (3.25 ms against 3.78 ms for ``dl @ w``), and d weight as
    ``acc += dl.t() @ xT.t()`` with ``xT`` the block's contiguous [H, n]
    hidden states (4.29 ms against 4.81 ms for ``acc += dl.t() @ x``).
    Other dtypes keep the plain forms."""

    def __init__(self, h2: Tensor, w: Tensor, need_h: bool, need_w: bool):
        self.w = w
        self.wide = w.dtype in (torch.bfloat16, torch.float16)
        self.dh = torch.zeros_like(h2, memory_format=torch.contiguous_format) if need_h else None
        self.wT = _transposed16(w) if (need_h and self.wide) else None
        self.dw = (torch.zeros(w.shape, dtype=torch.float32 if self.wide else w.dtype,
                               device=w.device) if need_w else None)

    def add_block(self, dl: Tensor, x_rows: Tensor, rows: Tensor) -> None:
        """dl [n, V] = d loss / d logits of the token rows ``rows``; x_rows
        their hidden states [n, H]."""

        if self.dh is not None:
            with nat.timed("lm_dhidden_gemm"):
                w = self.wT.t() if self.wT is not None else self.w
                self.dh.index_copy_(0, rows, torch.mm(dl, w))
        if self.dw is not None:
            with nat.timed("lm_dweight_gemm"):
                x = x_rows.t().contiguous().t() if self.wide else x_rows
                _addmm_into(self.dw, dl.t(), x)

    def finish(self) -> Tuple[Optional[Tensor], Optional[Tensor]]:
        dw = self.dw
        if dw is not None and dw.dtype != self.w.dtype:
            dw = dw.to(self.w.dtype)
        self.wT = None
        return self.dh, dw


def _logprob_rows(h2: Tensor, w: Tensor, tflat: Tensor, rows: Optional[Tensor], lse: Tensor,
                  logp: Tensor, status: Tensor, row_block: int) -> None:
    """lse and logp of the token rows ``rows`` (all when None), written into
    the [N] outputs: per row block the GEMM's logits, then rrl_logprob_fwd
    (the logits rounded to the weight dtype, as the reference's F.linear
    leaves them, for every token of the chunked path alike)."""

    dev = h2.device
    N = h2.shape[0]
    V = w.shape[0]
    n = N if rows is None else rows.numel()
    if n == 0:
        return
    x_all = h2 if rows is None else h2.index_select(0, rows)
    t_all = tflat if rows is None else tflat.index_select(0, rows)
    stream = nat.stream_ptr(dev)
    acc = lse.dtype
    blocks = _Blocks(w, row_block, n)
    lse_r = lse if rows is None else torch.empty(n, dtype=acc, device=dev)
    lp_r = logp if rows is None else torch.empty(n, dtype=acc, device=dev)
    for c0, c1 in blocks.spans(n):
        x = blocks.logits(x_all[c0:c1],
                          torch.arange(c0, c1, device=dev) if rows is None else rows[c0:c1])
        tv, _tk = nat.rows_view(t_all[c0:c1], 1, c1 - c0)
        nat.call("rrl_logprob_fwd", x.data_ptr(), nat.dtype_code(x.dtype), 1, c1 - c0, V, 0, V,
                 tv, lp_r[c0:].data_ptr(), nat.dtype_code(acc), lse_r[c0:].data_ptr(),
                 status.data_ptr(), stream)
    if rows is not None:
        lse.index_copy_(0, rows, lse_r)
        logp.index_copy_(0, rows, lp_r)


def _chunked_backward(h2: Tensor, w: Tensor, tflat: Tensor, lse: Tensor, logp: Tensor, g: Tensor,
                      need_h: bool, need_w: bool, row_block: int):
    """d hidden [N, H] and d weight [V, H] for d loss / d logp = g ([N], acc):
    the rows with g != 0 per row block: their logits again, dlogits written
    over them by rrl_logprob_bwd, then the two products."""

    dev = h2.device
    V = w.shape[0]
    grads = _Grads(h2, w, need_h, need_w)
    rows = torch.nonzero(g != 0).reshape(-1)
    n = rows.numel()
    if n:
        stream = nat.stream_ptr(dev)
        blocks = _Blocks(w, row_block, n)
        acc_code = nat.dtype_code(g.dtype)
        for c0, c1 in blocks.spans(n):
            idx = rows[c0:c1]
            xr = h2.index_select(0, idx)
            x = blocks.logits(xr, idx)
            tv, _tk = nat.rows_view(tflat.index_select(0, idx), 1, c1 - c0)
            lse_c = lse.index_select(0, idx)
            lp_c = logp.index_select(0, idx)
            g_c = g.index_select(0, idx)
            nat.call("rrl_logprob_bwd", x.data_ptr(), nat.dtype_code(x.dtype), 1, c1 - c0, V, 0, V,
                     tv, lse_c.data_ptr(), lp_c.data_ptr(), g_c.data_ptr(), x.data_ptr(),
                     nat.dtype_code(x.dtype), 0, V, 0, stream)
            del lse_c, lp_c, g_c
            grads.add_block(x, xr, idx)
    return grads.finish()


class _ChunkedLinearLogprobs(torch.autograd.Function):
    """log_softmax(hidden @ weight.T)[target] through row blocks of library
    GEMMs; the backward forms the logits of the rows with a non-zero gradient
    again.

    ``check``: the objective parameters whose target rule applies (any id
    outside [0, V) raises, as torch.gather does, except NLL's ignore_index,
    whose tokens get no target and log-prob 0).  ``weight_mask`` with
    ``skip_masked``: tokens of zero mask weight are not computed (log-prob 0);
    NLL passes labels != ignore_index, so ignored labels never are."""

    @staticmethod
    def forward(ctx, check: nat.RrlPolicyParams, skip_masked: bool, row_block: int,
                hidden: Tensor, weight: Tensor, target_ids: Tensor,
                weight_mask: Optional[Tensor] = None):
        dev = nat.require_device(hidden, weight, target_ids)
        B, T = _prepare(hidden, weight, target_ids)
        N, H = B * T, hidden.shape[-1]
        V = weight.shape[0]
        h2 = _rows2d(hidden, N, H)
        w = _rows2d(weight, V, H)
        tflat = target_ids.reshape(N)
        acc = nat.acc_dtype(hidden.dtype)
        status = nat.new_status(dev)
        tv, _keep = nat.rows_view(target_ids.reshape(B, T), B, T)
        nat.call("rrl_check_targets", L.ctypes_ref(check), B, T, V, tv, status.data_ptr(),
                 nat.stream_ptr(dev))
        L._raise_flags(nat.read_status(status) & nat.FLAG_TARGET_RANGE, check.kind)
        lse = torch.zeros(N, dtype=acc, device=dev)
        logp = torch.zeros(N, dtype=acc, device=dev)
        computed = None  # token rows whose lse exists (None: all)
        if weight_mask is None:
            _logprob_rows(h2, w, tflat, None, lse, logp, status, row_block)
        else:
            # The live tokens first, in the same row blocks with or without
            # skip_masked (a GEMM's rounding may depend on its block's other
            # rows), so that skipping the masked ones changes no live result.
            live = weight_mask.reshape(N) != 0
            _logprob_rows(h2, w, tflat, torch.nonzero(live).reshape(-1), lse, logp, status,
                          row_block)
            if not (skip_masked or check.kind == nat.OBJ_NLL):
                _logprob_rows(h2, w, tflat, torch.nonzero(~live).reshape(-1), lse, logp, status,
                              row_block)
            else:
                computed = live
        if nat.read_status(status) & nat.FLAG_TARGET_RANGE:
            L._raise_flags(nat.FLAG_TARGET_RANGE, check.kind)
        ctx.computed = computed
        ctx.save_for_backward(h2, w, tflat, lse, logp)
        ctx.meta = (hidden.shape, row_block)
        ctx.set_materialize_grads(False)
        return logp.view(hidden.shape[:-1])

    @staticmethod
    def backward(ctx, g):
        need_h, need_w = ctx.needs_input_grad[3], ctx.needs_input_grad[4]
        nones = (None, None, None)
        if g is None or not (need_h or need_w):
            return (*nones, None, None, None, None)
        h2, w, tflat, lse, logp = ctx.saved_tensors
        shape, row_block = ctx.meta
        gc = g.reshape(-1).to(lse.dtype).contiguous()
        if ctx.computed is not None:
            # an ignored label or a skipped token has a constant log-prob: no
            # gradient, whatever the upstream gradient holds there
            gc = torch.where(ctx.computed, gc, torch.zeros((), dtype=gc.dtype, device=gc.device))
        dh, dw = _chunked_backward(h2, w, tflat, lse, logp, gc, need_h, need_w, row_block)
        return (*nones, (dh.view(shape) if dh is not None else None), dw, None, None)


class _ChunkedLinearPolicy(torch.autograd.Function):
    """A token-local objective (PPO/GRPO clip, SAO, SAPO) behind the LM head
    in one sweep per row block of active tokens: logits (GEMM), then
    rrl_fused_logprob_policy (log-prob, lse, dlogits over the logits for an
    upstream d loss = 1), then the d hidden rows and the block's share of
    d weight (GEMMs).  Tokens of zero mask weight take the log-sum-exp pass
    only (log-prob 0 with ``skip_masked``).  Without gradients every token
    takes that pass.  The backward rescales the stored gradients when
    autograd hands another scale, and runs the general chunked backward when
    diagnostics also receive gradients.  Outputs as ``_FusedPolicy``."""

    @staticmethod
    def forward(ctx, params: nat.RrlPolicyParams, opts: Tuple[bool, bool], row_block: int,
                hidden: Tensor, weight: Tensor, target_ids: Tensor, old: Tensor, adv: Tensor,
                mask: Tensor):
        # opts: (skip_masked, the caller's grad mode; forward itself runs with
        # grad mode off)
        skip_masked, grad_mode = opts
        kind = params.kind
        dev = nat.require_device(hidden, weight, target_ids, old, adv, mask)
        B, T = _prepare(hidden, weight, target_ids)
        N, H = B * T, hidden.shape[-1]
        V = weight.shape[0]
        h2 = _rows2d(hidden, N, H)
        w = _rows2d(weight, V, H)
        acc = nat.acc_dtype(hidden.dtype, old.dtype, adv.dtype)
        acc_code = nat.dtype_code(acc)
        stream = nat.stream_ptr(dev)
        pref = L.ctypes_ref(params)
        tview, tkeep = nat.rows_view(target_ids, B, T)
        ov, ok = nat.rows_view(old, B, T)
        av, ak = nat.rows_view(adv, B, T)
        mv, mk = nat.rows_view(mask, B, T)
        ws = torch.empty(nat.lib().rrl_policy_workspace_bytes(B, acc_code), dtype=torch.uint8,
                         device=dev)
        coef = torch.empty(B, dtype=acc, device=dev)
        status = nat.new_status(dev)
        # Every data error is known before the sweep: the row coefficients flag
        # empty masks, rrl_check_targets the targets.
        nat.call("rrl_policy_row_coef", pref, B, T, mv, acc_code, coef.data_ptr(), ws.data_ptr(),
                 status.data_ptr(), stream)
        nat.call("rrl_check_targets", pref, B, T, V, tview, status.data_ptr(), stream)
        L._raise_flags(nat.read_status(status), kind)

        need_h, need_w = ctx.needs_input_grad[3], ctx.needs_input_grad[4]
        eager = grad_mode and (need_h or need_w)
        tflat = tkeep.reshape(N)
        lse = torch.zeros(N, dtype=acc, device=dev)
        logp = torch.zeros(N, dtype=acc, device=dev)
        grads = None
        if eager:
            live = mk.reshape(N) != 0
            act = torch.nonzero(live).reshape(-1)
            if not skip_masked:
                _logprob_rows(h2, w, tflat, torch.nonzero(~live).reshape(-1), lse, logp, status,
                              row_block)
            grads = _ChunkedLinearPolicy._sweep(params, h2, w, tflat, ok, ak, mk, coef, act, T,
                                                lse, logp, need_h, need_w, row_block, status)
            flags = nat.read_status(status)
            if flags & nat.FLAG_FAST_RANGE:
                # A row's log-sum-exp beyond the register-resident kernel's
                # exponent range (bf16 logits near 2e38): redo the sweep on the
                # generic row kernel (the block's logits were overwritten).
                generic = nat.RrlPolicyParams.from_buffer_copy(params)
                generic.flags |= nat.POLICY_GENERIC
                status.zero_()
                grads = _ChunkedLinearPolicy._sweep(generic, h2, w, tflat, ok, ak, mk, coef, act,
                                                    T, lse, logp, need_h, need_w, row_block,
                                                    status)
        else:
            live = mk.reshape(N) != 0
            _logprob_rows(h2, w, tflat, torch.nonzero(live).reshape(-1), lse, logp, status,
                          row_block)
            if not skip_masked:
                _logprob_rows(h2, w, tflat, torch.nonzero(~live).reshape(-1), lse, logp, status,
                              row_block)
        scal = torch.empty(nat.NSCALARS, dtype=acc, device=dev)
        trusted = torch.empty(N if kind == nat.OBJ_SAO else 0, dtype=torch.bool, device=dev)
        lview = nat.RrlView(logp.data_ptr(), acc_code, T, 1)
        nat.call("rrl_policy_fwd", pref, B, T, lview, ov, av, mv, acc_code, ws.data_ptr(),
                 scal.data_ptr(), None, nat.ptr(trusted) if trusted.numel() else None,
                 status.data_ptr(), stream)
        L._raise_flags(nat.read_status(status) & ~nat.FLAG_FAST_RANGE, kind)

        ctx.params = params
        ctx.grads = grads
        ctx.meta = (B, T, acc, hidden.shape, row_block)
        ctx.save_for_backward(h2, w, tflat, ok, ak, mk, lse, logp, ws)
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
    def _sweep(params, h2, w, tflat, ok, ak, mk, coef, act, T, lse, logp, need_h, need_w,
               row_block, status):
        """The single sweep over the active rows ``act``, in row blocks."""

        dev = h2.device
        N = h2.shape[0]
        V = w.shape[0]
        stream = nat.stream_ptr(dev)
        pref = L.ctypes_ref(params)
        grads = _Grads(h2, w, need_h, need_w)
        n = act.numel()
        if n == 0:
            return grads.finish()
        blocks = _Blocks(w, row_block, n)
        acc = lse.dtype
        oflat, aflat, mflat = ok.reshape(N), ak.reshape(N), mk.reshape(N)
        seq_of = act // T
        dt = nat.dtype_code(w.dtype)
        records = torch.empty(nat.lib().rrl_fused_records_bytes(blocks.cap, 1), dtype=torch.uint8,
                              device=dev)
        lp_c = torch.empty(blocks.cap, dtype=acc, device=dev)
        lse_c = torch.empty(blocks.cap, dtype=acc, device=dev)
        for c0, c1 in blocks.spans(n):
            idx = act[c0:c1]
            m = c1 - c0
            xr = h2.index_select(0, idx)
            x = blocks.logits(xr, idx)
            # one token per row: [m, 1] views of the block's side data
            tv, tk = nat.rows_view(tflat.index_select(0, idx), m, 1)
            ov, okb = nat.rows_view(oflat.index_select(0, idx), m, 1)
            av, akb = nat.rows_view(aflat.index_select(0, idx), m, 1)
            mv, mkb = nat.rows_view(mflat.index_select(0, idx), m, 1)
            cc = coef.index_select(0, seq_of[c0:c1])
            nat.call("rrl_fused_logprob_policy", pref, x.data_ptr(), dt, m, 1, V, V, V, tv, ov,
                     av, mv, cc.data_ptr(), records.data_ptr(), lp_c.data_ptr(),
                     lse_c.data_ptr(), x.data_ptr(), dt, V, V, status.data_ptr(), stream)
            logp.index_copy_(0, idx, lp_c[:m])
            lse.index_copy_(0, idx, lse_c[:m])
            grads.add_block(x, xr, idx)
            del tk, okb, akb, mkb, cc
        return grads.finish()

    @staticmethod
    def backward(ctx, g0, g1, g2, g3, _glogp, _gtrusted):
        need_h, need_w = ctx.needs_input_grad[3], ctx.needs_input_grad[4]
        nones = (None, None, None)
        if not (need_h or need_w):
            return (*nones, None, None, None, None, None, None)
        B, T, acc, shape, row_block = ctx.meta
        params = ctx.params
        h2, w, tflat, ok, ak, mk, lse, logp, ws = ctx.saved_tensors
        dev = lse.device
        stream = nat.stream_ptr(dev)
        grads = ctx.grads
        extra = any(g is not None for g in (g1, g3)) or (
            params.kind == nat.OBJ_SAPO and g2 is not None)
        if grads is not None and not extra:
            # the stored gradients are those of d(-objective) = d loss
            scale = (-g0).reshape(1).to(acc) if g0 is not None else torch.zeros(
                1, dtype=acc, device=dev)
            dh, dw = grads
            out = []
            for t in (dh, dw):
                if t is not None:
                    rows, width = t.shape
                    nat.call("rrl_scale_rows", t.data_ptr(), nat.dtype_code(t.dtype), 1, rows,
                             width, 0, width, scale.data_ptr(), nat.dtype_code(acc), 1.0, stream)
                out.append(t)
            ctx.grads = None
            dh, dw = out
            return (*nones, (dh.view(shape) if dh is not None and need_h else None),
                    dw if need_w else None, None, None, None, None)
        # General case: d loss / d logp from every differentiated output, then
        # the chunked backward over the rows it reaches.
        gs = torch.zeros(nat.NSCALARS, dtype=acc, device=dev)
        for k, g in enumerate((g0, g1, g2, g3)):
            if g is not None:
                gs[k] = g.to(acc)
        lview = nat.RrlView(logp.data_ptr(), nat.dtype_code(acc), T, 1)
        ov, _ = nat.rows_view(ok, B, T)
        av, _ = nat.rows_view(ak, B, T)
        mv, _ = nat.rows_view(mk, B, T)
        g = torch.empty(B * T, dtype=acc, device=dev)
        nat.call("rrl_policy_bwd", L.ctypes_ref(params), B, T, lview, ov, av, mv,
                 nat.dtype_code(acc), ws.data_ptr(), gs.data_ptr(), None, g.data_ptr(), stream)
        ctx.grads = None
        dh, dw = _chunked_backward(h2, w, tflat, lse, logp, g, need_h, need_w, row_block)
        return (*nones, (dh.view(shape) if dh is not None else None), dw, None, None, None, None)


# ---------------------------------------------------------------------------
# Tile path: hand-written MFMA kernels, no logits beyond one tile
# ---------------------------------------------------------------------------


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
    """log_softmax(hidden @ weight.T)[target] on the hand-written matrix-core
    kernels; the forward keeps obar for d hidden, the backward recomputes
    logits tiles for d W.

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
        computed = None  # token rows whose lse exists (None: all)
        if need and weight_mask is not None:
            live = weight_mask.reshape(N) != 0
            if skip_masked:
                need_rows = torch.where(live, 1, 2).to(torch.uint8).contiguous()
                computed = live
            else:
                need_rows = live.to(torch.uint8).contiguous()
        lse, logp, obar, flags = lm_head_forward(h2, w, tgt32, need, status, need_rows)
        if flags & nat.FLAG_TARGET_RANGE:
            L._raise_flags(nat.FLAG_TARGET_RANGE, check.kind)
        ctx.save_for_backward(h2, w, tgt32, lse, logp, obar)
        ctx.computed = computed
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
        if ctx.computed is not None:
            # a skipped token's log-prob is the constant 0: no gradient (its
            # lse and obar were never formed); ignored labels (target -1) are
            # left out by the kernels themselves
            gc = torch.where(ctx.computed, gc, torch.zeros((), dtype=gc.dtype, device=gc.device))
        dh, dw = lm_head_backward(h2, w, tgt32, lse, logp, obar, gc, need_h, need_w)
        return (None, (dh.view(ctx.hidden_shape) if dh is not None else None), dw, None, None,
                None)


# ---------------------------------------------------------------------------
# Public API
# ---------------------------------------------------------------------------


def _linear_logprobs(check: nat.RrlPolicyParams, impl: str, row_block: int, hidden: Tensor,
                     weight: Tensor, target_ids: Tensor, weight_mask: Optional[Tensor] = None,
                     skip_masked: bool = False) -> Tensor:
    _prepare(hidden, weight, target_ids)
    if _resolve_impl(impl, hidden) == "tiles":
        return _LinearLogprobs.apply(check, hidden, weight, target_ids, weight_mask, skip_masked)
    return _ChunkedLinearLogprobs.apply(check, bool(skip_masked), int(row_block), hidden, weight,
                                        target_ids, weight_mask)


def linear_token_logprobs(hidden: Tensor, weight: Tensor, target_ids: Tensor, *,
                          row_block: int = DEFAULT_ROW_BLOCK, impl: str = "auto") -> Tensor:
    """``gather_token_logprobs(hidden @ weight.T, target_ids)`` without the
    whole logits tensor.

    ``hidden``: [..., H]; ``weight``: [V, H] (an LM head without bias, tied or
    not), one float dtype; ``target_ids``: hidden's prefix shape.  Returns
    log-probs in float32 (float64 for float64 inputs), as
    ``gather_token_logprobs`` does for 16-bit logits.  Differentiable into
    ``hidden`` and ``weight``.  ``impl="chunked"`` (``"auto"``) holds at most
    ``row_block`` rows of logits at a time; ``impl="tiles"`` (bfloat16, H a
    multiple of 128 up to 1024) none beyond a 32 x 64 tile.
    """

    _check_row_block(row_block)
    return _cfg.as_reference_dtype(
        _linear_logprobs(L._params(nat.OBJ_PPO), impl, row_block, hidden, weight, target_ids),
        hidden)


def linear_label_logprobs(hidden: Tensor, weight: Tensor, labels: Tensor, ignore_index: int, *,
                          row_block: int = DEFAULT_ROW_BLOCK, impl: str = "auto") -> Tensor:
    """:func:`linear_token_logprobs` for cross-entropy labels: a label equal to
    ``ignore_index`` has no target (log-prob 0, no gradient) and is exempt
    from the range check, whose failure raises IndexError as F.cross_entropy
    does."""

    p = nat.RrlPolicyParams()
    p.kind = nat.OBJ_NLL
    p.ignore_index = int(ignore_index)
    _check_row_block(row_block)
    return _linear_logprobs(p, impl, row_block, hidden, weight, labels,
                            labels != int(ignore_index))


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
    impl: str = "auto",
):
    """``fused_policy_loss(hidden @ weight.T, ...)`` without the whole logits
    tensor.

    ``hidden``: [..., H] final hidden states at the positions that predict
    ``target_ids`` (already shifted); ``weight``: the LM head's [V, H] weight
    (no bias).  Objectives and options as :func:`fused_policy_loss`; the loss
    is differentiable into ``hidden`` and ``weight``.

    ``impl="chunked"`` (``"auto"``): row blocks of at most ``row_block``
    tokens; for the token-local objectives one sweep per block of active
    tokens forms their logits once and writes both gradients' shares then and
    there (d hidden, d weight for an upstream d loss = 1, rescaled by the
    backward).  ``impl="tiles"``: the hand-written MFMA kernels (bfloat16,
    H a multiple of 128 up to 1024; no logits beyond one tile).

    ``skip_masked_rows=True`` (a training step, with gradients asked for)
    leaves out the tokens whose mask weight is 0 (the tile path: every block
    of 64 such consecutive tokens): their log-probs are taken as 0, which a
    masked token's term multiplies by 0, so the loss and the gradients are
    those of the full computation, without the log-sum-exp pass over those
    tokens (no reference counterpart).
    """

    if objective not in L._OBJECTIVES:
        raise ValueError(
            f"unknown objective {objective!r}; expected one of {sorted(L._OBJECTIVES)}")
    kind = L._OBJECTIVES[objective]
    _prepare(hidden, weight, target_ids)
    if skip_masked_rows and return_logprobs:
        raise ValueError("skip_masked_rows=True leaves masked log-probs uncomputed; "
                         "it cannot be combined with return_logprobs=True")
    _check_row_block(row_block)
    path = _resolve_impl(impl, hidden)
    mask = L._on_device(action_mask, hidden)
    ppo = L._params(nat.OBJ_PPO)
    if kind in (nat.OBJ_GSPO, nat.OBJ_GSPO_TOKEN):
        logp = _linear_logprobs(ppo, path, row_block, hidden, weight, target_ids,
                                mask.expand(target_ids.shape), bool(skip_masked_rows))
        fn = L.gspo_policy_loss if kind == nat.OBJ_GSPO else L.gspo_token_policy_loss
        out = fn(logp, old_logprobs, advantages, action_mask, clip_low=clip_low,
                 clip_high=clip_low if clip_high is None else clip_high,
                 max_log_ratio=max_log_ratio)
        return (out, _cfg.as_reference_dtype(logp.detach(), hidden)) if return_logprobs else out

    p = L._token_local_params(kind, hidden.shape[:-1], old_logprobs, advantages, action_mask,
                              clip_low=clip_low, clip_high=clip_high,
                              max_log_ratio=max_log_ratio, detach_ratio=detach_ratio,
                              tau_positive=tau_positive, tau_negative=tau_negative)
    if path == "tiles":
        logp = _LinearLogprobs.apply(ppo, hidden, weight, target_ids, mask,
                                     bool(skip_masked_rows))
        obj, d1, d2, d3, _seq, trusted = L._objective(p, logp, old_logprobs, advantages, mask)
        out = L._token_local_output(kind, obj, d1, d2, d3, trusted)
        return (out, _cfg.as_reference_dtype(logp.detach(), hidden)) if return_logprobs else out
    prefix = hidden.shape[:-1]
    old_d = L._on_device(old_logprobs, hidden)
    adv_d = L._on_device(advantages, hidden)
    obj, d1, d2, d3, logp, trusted = _ChunkedLinearPolicy.apply(
        p, (bool(skip_masked_rows), torch.is_grad_enabled()), int(row_block), hidden, weight,
        target_ids,
        old_d.expand(prefix), adv_d.expand(prefix), mask.expand(prefix))
    out = L._token_local_output(kind, obj, d1, d2, d3, trusted)
    return (out, _cfg.as_reference_dtype(logp, hidden)) if return_logprobs else out
