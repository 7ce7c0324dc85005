"""HIP path vs the CPU oracle on identical seeded inputs (MI355X).

Tolerances (north star): float32 results within 1e-5 relative, bf16-input
log-probs and losses within 2e-3 relative.  16-bit dlogits: every element
within one ulp of the correctly rounded exact value (at least 98% of them
bit-identical to it), and each row within 2e-3 norm-wise relative error of
that correctly rounded row.  The rounded row is the reference point because
bf16's unit roundoff is 2^-8 = 3.9e-3: a correctly rounded row whose norm is
carried by one element (the target column) can itself sit 3.5e-3 from the
exact values, and f16 flushes whole rows of ~1e-9 gradients to zero.  Log-probs and dlogits are held against the
float64 evaluation of the reference's math on exact upcasts of the same
inputs (``exact=True``): a float32 evaluation, the reference's own, carries
cancellation error of several float32 ulps of the row log-sum-exp where
log p -> 0, which a 1e-5 relative bound cannot absorb.
Index, mask and alignment outputs are compared bit-exactly, except decisions
whose oracle ratio sits within float32 rounding of a threshold (excluded by
distance, reported by count).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import roserlhf_oracle as o
from rosellm_amd import roserlhf as R
from rosellm_amd.roserlhf import losses as L

pytestmark = pytest.mark.gpu

F32_RTOL = 1e-5


def _close(got, want, rtol, atol, what=""):
    got = got.detach().double().cpu()
    want = want.detach().double().cpu()
    assert got.shape == want.shape, (what, got.shape, want.shape)
    err = (got - want).abs()
    bound = atol + rtol * want.abs()
    bad = ~(err <= bound) & ~(torch.isnan(got) & torch.isnan(want))
    if bad.any():
        excess = torch.where(bad, err / bound.clamp_min(1e-300), torch.zeros_like(err))
        i = int(excess.reshape(-1).argmax())
        idx = np.unravel_index(i, tuple(got.shape)) if got.dim() else ()
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {got.numel()} outside tol; worst at {idx}: "
            f"got {got.reshape(-1)[i].item():.9g} want {want.reshape(-1)[i].item():.9g} "
            f"(err {err.reshape(-1)[i].item():.3e}, bound {bound.reshape(-1)[i].item():.3e})"
        )


def _rownorm(got, want, tol, what=""):
    g = got.detach().double().cpu().reshape(-1, got.shape[-1])
    w = want.detach().double().cpu().reshape(-1, want.shape[-1])
    num = (g - w).norm(dim=-1)
    den = w.norm(dim=-1)
    rel = torch.where(den > 0, num / den.clamp_min(1e-30), num)
    assert rel.max().item() <= tol, f"{what}: worst row-norm rel err {rel.max().item():.3e}"
    return rel.max().item()


def _rownorm16(got, want_exact, tol=2e-3, what=""):
    """16-bit rows against the correctly rounded exact rows (see module doc);
    prints the distance to the unrounded values for the record."""

    rounded = want_exact.detach().cpu().float().to(got.dtype)
    worst = _rownorm(got, rounded, tol, what)
    g = got.detach().double().cpu().reshape(-1, got.shape[-1])
    w = want_exact.detach().double().cpu().reshape(-1, got.shape[-1])
    den = w.norm(dim=-1)
    vs_exact = torch.where(den > 0, (g - w).norm(dim=-1) / den.clamp_min(1e-30), den * 0)
    print(f"{what}: worst row-norm rel err vs rounded {worst:.3e}, vs exact "
          f"{vs_exact.max().item():.3e}", flush=True)
    return worst


def _close_rows_by_g(got, want, g, rtol, what=""):
    """dlogits[row] = g * (onehot - softmax): every element's float32 error is
    bounded by a few ulp of |g| (1 - p_target cancels when p_target -> 1), so
    each row is compared relative to its upstream gradient |d loss / d logp|."""

    e = (got.detach().double().cpu() - want.detach().double().cpu()).abs()
    e = e.reshape(-1, e.shape[-1]).max(dim=-1).values
    bound = rtol * g.detach().double().cpu().reshape(-1).abs() + 1e-12
    bad = e > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} rows beyond {rtol}*|g|; worst {(e / bound).max():.2f}x"


def _ord16(t):
    """Order-preserving integer image of 16-bit float bit patterns."""

    b = t.contiguous().view(torch.int16).to(torch.int32)
    return torch.where(b < 0, -(b & 0x7FFF), b)


def _ulp16(got, want_f32, what=""):
    """16-bit outputs: each element within 1 ulp of the correctly rounded
    (round-to-nearest-even) oracle value; returns the fraction bit-identical
    to it.  One ulp covers float32 error at rounding midpoints; the
    worst-case relative error of any bf16 result is 2^-8 of the value."""

    g = got.detach().cpu()
    w = want_f32.detach().cpu().float().to(got.dtype)
    dist = (_ord16(g) - _ord16(w)).abs()
    tiny = (g.float() - want_f32.detach().cpu().float()).abs() < 1e-30
    bad = (dist > 1) & ~tiny
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond 1 ulp (max {int(dist.max())})"
    return (dist == 0).float().mean().item()


def _gen(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------------------
# a1/a2 log-probs
# ---------------------------------------------------------------------------


@pytest.mark.parametrize(
    "dtype,V,B,T",
    [
        (torch.float32, 50257, 2, 6),  # config-1 vocab: rows not 16-byte aligned
        (torch.bfloat16, 151936, 2, 5),  # config-2 vocab
        (torch.float16, 4099, 3, 4),
        (torch.float64, 1001, 2, 3),
        (torch.float32, 7, 1, 3),  # vocab smaller than one vector
        (torch.bfloat16, 1, 2, 2),  # single-entry vocabulary
    ],
)
def test_logprob_forward_backward(device, dtype, V, B, T):
    print(f"[logprob] dtype={dtype} V={V} B={B} T={T}", flush=True)
    g = _gen(V + B)
    x = (torch.randn(B, T, V, generator=g) * 3.0).to(dtype)
    if V > 4:
        x[0, 0, 3] = 15.0  # dominant logit
        x[-1, -1, : V // 2] = -float("inf")  # masked vocabulary
    t = torch.randint(0, V, (B, T), generator=g)
    if V > 4:
        t[-1, -1] = V - 1
    up = torch.randn(B, T, generator=g, dtype=torch.float64)

    xd = x.to(device).requires_grad_()
    lp = R.gather_token_logprobs(xd, t.to(device))
    acc = torch.float64 if dtype == torch.float64 else torch.float32
    assert lp.dtype == acc
    xo = x.double().requires_grad_()
    lpo = o.token_logprobs(xo, t, exact=True)
    rtol = 1e-12 if dtype == torch.float64 else F32_RTOL
    _close(lp, lpo, rtol, 1e-7 if dtype != torch.float64 else 1e-12, "logp")

    (lp * up.to(device).to(acc)).sum().backward()
    (lpo * up).sum().backward()
    dl, dlo = xd.grad, xo.grad
    assert dl.dtype == dtype and dl.shape == x.shape
    if dtype in (torch.bfloat16, torch.float16):
        exact = _ulp16(dl, dlo, "dlogits")
        assert exact > 0.98, exact
        _rownorm16(dl, dlo, 2e-3, "dlogits")
    elif dtype == torch.float64:
        _close(dl, dlo, 1e-12, 1e-14, "dlogits")
    else:
        _close_rows_by_g(dl, dlo, up, F32_RTOL, "dlogits")


def test_logprob_causal_shift_views(device):
    """logits[:, :-1] with input_ids[:, 1:] (source-lab.md:139-147) is read in place."""

    g = _gen(3)
    B, S, V = 3, 9, 333
    x = torch.randn(B, S, V, generator=g)
    ids = torch.randint(0, V, (B, S), generator=g)
    xd = x.to(device).requires_grad_()
    lp = R.gather_token_logprobs(xd[:, :-1], ids.to(device)[:, 1:])
    xo = x.double().requires_grad_()
    lpo = o.token_logprobs(xo[:, :-1], ids[:, 1:], exact=True)
    _close(lp, lpo, F32_RTOL, 1e-7, "shifted logp")
    lp.sum().backward()
    lpo.sum().backward()
    _close(xd.grad, xo.grad, F32_RTOL, 1e-7, "shifted dlogits")


def test_logprob_int32_targets_and_rank2(device):
    g = _gen(4)
    x = torch.randn(17, 129, generator=g)
    t = torch.randint(0, 129, (17,), generator=g, dtype=torch.int32)
    lp = R.gather_token_logprobs(x.to(device), t.to(device))
    _close(lp, o.token_logprobs(x, t, exact=True), F32_RTOL, 1e-7, "rank-2 logp")


def test_logprob_target_out_of_range_raises(device):
    x = torch.randn(2, 3, 10, device=device)
    t = torch.zeros(2, 3, dtype=torch.long, device=device)
    t[1, 2] = 10
    with pytest.raises(RuntimeError, match="out of bounds"):
        R.gather_token_logprobs(x, t)


@pytest.mark.parametrize("tdtype", [torch.int64, torch.int32])
def test_check_targets_through_the_c_abi(device, tdtype):
    """rrl_check_targets flags TARGET_RANGE for any id outside [0, V) except
    NLL's ignore_index, on strided views too, and never for valid ids."""

    from rosellm_amd import _native as nat
    from rosellm_amd.rosetrainer import lm_loss as LM

    B, T, V = 5, 300, 1000
    wide = torch.randint(0, V, (B, T + 3), device=device, dtype=tdtype)
    view = wide[:, 1:T + 1]

    def flags(t, params):
        st = torch.zeros(1, dtype=torch.int32, device=device)
        tv, _keep = nat.rows_view(t, B, T)
        nat.call("rrl_check_targets", L.ctypes_ref(params), B, T, V, tv, st.data_ptr(),
                 nat.stream_ptr(device))
        return int(st.item())

    ppo = L._params(nat.OBJ_PPO, clip_low=0.2, clip_high=0.2)
    nll = LM._nll_params(-100, "mean")
    assert flags(view, ppo) == 0 and flags(view, nll) == 0
    wide[0, 0] = V  # outside the view: not checked
    assert flags(view, ppo) == 0
    for badv in (V, -1, -100):
        w2 = wide.clone()
        w2[3, 17] = badv
        want = 0 if (badv == -100) else nat.FLAG_TARGET_RANGE
        assert flags(w2[:, 1:T + 1], ppo) == nat.FLAG_TARGET_RANGE
        assert flags(w2[:, 1:T + 1], nll) == want


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16, torch.bfloat16])
def test_fused_data_errors_raise(device, dtype):
    """Out-of-range targets, an empty mask and SAPO's empty rows raise the
    reference's errors whether the status is read before the sweep (every
    dtype out of place) or after it (bfloat16 in place); a valid call right
    after works."""

    B, T, V = 4, 6, 4096
    x, t, old, adv, mask = _fused_inputs(71, B, T, V, dtype)
    d = lambda v: v.to(device)  # noqa: E731
    for badv in (V, -1):
        bad = t.clone()
        bad[2, 3] = badv
        with pytest.raises(RuntimeError, match="out of bounds"):
            R.fused_policy_loss(d(x), d(bad), d(old), d(adv), d(mask))
        with pytest.raises(RuntimeError, match="out of bounds"):
            R.fused_policy_loss(d(x), d(bad), d(old), d(adv), d(mask), inplace=True)
    with pytest.raises(ValueError, match="empty mask"):
        R.fused_policy_loss(d(x), d(t), d(old), d(adv), d(torch.zeros_like(mask)))
    rows = mask.clone()
    rows[1] = False
    with pytest.raises(ValueError, match="at least one action token"):
        R.fused_policy_loss(d(x), d(t), d(old), d(adv), d(rows), objective="sapo")
    xd = d(x).requires_grad_()
    out = R.fused_policy_loss(xd, d(t), d(old), d(adv), d(mask), clip_low=0.2, clip_high=0.28)
    out.loss.backward()
    out_o, _, dlo = o.policy_step("ppo", x, t, old, adv, mask, exact=True, clip_low=0.2,
                                  clip_high=0.28)
    scale = max(abs(float(out_o["loss"])), float(adv.abs().mean()))
    assert abs(out.loss.item() - float(out_o["loss"])) <= 2e-3 * scale
    _rownorm16(xd.grad, dlo, 2e-3, "dlogits after the errors")


def test_logprob_empty(device):
    x = torch.randn(0, 4, 11, device=device, requires_grad=True)
    t = torch.zeros(0, 4, dtype=torch.long, device=device)
    lp = R.gather_token_logprobs(x, t)
    assert lp.shape == (0, 4)
    lp.sum().backward()
    assert x.grad.shape == x.shape


# ---------------------------------------------------------------------------
# objectives
# ---------------------------------------------------------------------------


def _policy_inputs(seed, B=6, T=40, dtype=torch.float32):
    """Random log-probs; ratio exactly 1 at (0, 0..2) (exp(0) is exact on every
    device, so clip_low/clip_high = 0 put it exactly on a boundary) and a
    log-ratio beyond the clamp at (1, 0)."""

    g = _gen(seed)
    old = -torch.rand(B, T, generator=g, dtype=torch.float64) * 6.0
    cur = old + torch.randn(B, T, generator=g, dtype=torch.float64) * 0.2
    cur[0, :3] = old[0, :3]
    cur[1, 0] = old[1, 0] + 25.0  # beyond max_log_ratio
    adv = torch.randn(B, T, generator=g, dtype=torch.float64)
    adv[2, :4] = 0.0
    mask = torch.rand(B, T, generator=g) < 0.75
    mask[:, 0] = True
    return cur.to(dtype), old.to(dtype), adv.to(dtype), mask


def _run_both(fn_hip, fn_oracle, cur, old, adv, mask, device, diag_names, **kw):
    c_h = cur.to(device).requires_grad_()
    out_h = fn_hip(c_h, old.to(device), adv.to(device), mask.to(device), **kw)
    c_o = cur.clone().requires_grad_()
    out_o = fn_oracle(c_o, old, adv, mask, **kw)
    return c_h, out_h, c_o, out_o


def _check_scalars(out_h, out_o, names, rtol, atol):
    for n in names:
        _close(getattr(out_h, n).reshape(-1), out_o[n].reshape(-1), rtol, atol, n)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("mask_kind", ["bool", "float", "int"])
def test_clipped_policy_loss_parity(device, dtype, mask_kind):
    cur, old, adv, mask = _policy_inputs(11, dtype=dtype)
    m = {"bool": mask, "float": mask.to(dtype) * 0.5, "int": mask.long()}[mask_kind]
    kw = dict(clip_low=0.2, clip_high=0.28)
    c_h, out_h, c_o, out_o = _run_both(R.clipped_policy_loss, o.ppo_clip, cur, old, adv, m,
                                       device, None, **kw)
    rtol, atol = (1e-12, 1e-14) if dtype == torch.float64 else (F32_RTOL, 1e-7)
    _check_scalars(out_h, out_o, ["loss", "objective", "approximate_kl", "clip_fraction",
                                  "mean_ratio"], rtol, atol)
    # gradient through the loss and through the differentiable diagnostics
    (out_h.loss + 0.3 * out_h.approximate_kl - 0.7 * out_h.mean_ratio).backward()
    (out_o["loss"] + 0.3 * out_o["approximate_kl"] - 0.7 * out_o["mean_ratio"]).backward()
    _close(c_h.grad, c_o.grad, rtol, atol, "grad")
    assert out_h.clip_fraction.requires_grad is False


@pytest.mark.parametrize("clip", [(0.0, 0.2), (0.2, 0.0), (0.0, 0.0)])
def test_exact_boundary_ratios(device, clip):
    """Ratio exactly 1 on a clip / trust boundary: clamp passes gradient on the
    closed band, minimum splits ties, DIS trust is strict (losses.py:124, :465-470)."""

    cur, old, adv, mask = _policy_inputs(40)
    adv[0, 0], adv[0, 1], adv[0, 2] = 1.0, -1.0, 0.0
    lo_eps, hi_eps = clip
    for fn_h, fn_o, kw in (
        (R.clipped_policy_loss, o.ppo_clip, dict(clip_low=lo_eps, clip_high=hi_eps)),
        (R.sao_policy_loss, o.sao, dict(clip_low=lo_eps, clip_high=hi_eps)),
    ):
        c_h, out_h, c_o, out_o = _run_both(fn_h, fn_o, cur, old, adv, mask, device, None, **kw)
        out_h.loss.backward()
        out_o["loss"].backward()
        _close(c_h.grad, c_o.grad, F32_RTOL, 1e-7, f"{fn_h.__name__} {clip} grad")
        _close(out_h.loss, out_o["loss"], F32_RTOL, 1e-7, f"{fn_h.__name__} {clip} loss")
        if fn_h is R.sao_policy_loss:
            assert torch.equal(out_h.trusted_mask.cpu(), out_o["trusted_mask"])


def test_clipped_policy_loss_strided_advantages(device):
    """Advantages broadcast with expand() (examples/agentic_rl_toy.py:106) are read in place."""

    cur, old, _, mask = _policy_inputs(12)
    seq_adv = torch.randn(cur.shape[0], generator=_gen(1))
    adv_h = seq_adv.to(device)[:, None].expand(cur.shape)
    c_h = cur.to(device).requires_grad_()
    out_h = R.clipped_policy_loss(c_h, old.to(device), adv_h, mask.to(device), clip_low=0.2)
    c_o = cur.clone().requires_grad_()
    out_o = o.ppo_clip(c_o, old, seq_adv[:, None].expand(cur.shape), mask, clip_low=0.2)
    _close(out_h.loss, out_o["loss"], F32_RTOL, 1e-7, "loss")
    out_h.loss.backward()
    out_o["loss"].backward()
    _close(c_h.grad, c_o.grad, F32_RTOL, 1e-7, "grad")


def _threshold_safe(ratio, lo, hi, rel=1e-6):
    return ((ratio - lo).abs() > rel * lo) & ((ratio - hi).abs() > rel * hi)


@pytest.mark.parametrize("detach", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_sao_parity(device, detach, dtype):
    cur, old, adv, mask = _policy_inputs(13, dtype=dtype)
    kw = dict(clip_low=0.2, clip_high=0.28, detach_ratio=detach)
    c_h, out_h, c_o, out_o = _run_both(R.sao_policy_loss, o.sao, cur, old, adv, mask, device,
                                       None, **kw)
    rtol, atol = (1e-12, 1e-14) if dtype == torch.float64 else (F32_RTOL, 1e-7)
    ratio = torch.exp((cur - old).clamp(-20, 20)).double()
    safe = _threshold_safe(ratio, 0.8, 1.28)
    th, to = out_h.trusted_mask.cpu(), out_o["trusted_mask"]
    assert torch.equal(th[safe], to[safe]), "trusted mask differs away from thresholds"
    if dtype == torch.float64:
        assert torch.equal(th, to)
    _check_scalars(out_h, out_o, ["loss", "approximate_kl", "rejected_fraction", "mean_ratio"],
                   rtol, atol)
    (out_h.loss + 0.25 * out_h.approximate_kl + out_h.mean_ratio).backward()
    (out_o["loss"] + 0.25 * out_o["approximate_kl"] + out_o["mean_ratio"]).backward()
    _close(c_h.grad, c_o.grad, rtol, atol, "grad")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_gspo_parity(device, dtype):
    cur, old, _, mask = _policy_inputs(14, dtype=dtype)
    cur[1, 0] = old[1, 0] + 0.01  # keep the sequence ratios moderate
    seq_adv = torch.randn(cur.shape[0], generator=_gen(2), dtype=dtype)
    kw = dict(clip_low=3e-4, clip_high=4e-4)
    c_h = cur.to(device).requires_grad_()
    out_h = R.gspo_policy_loss(c_h, old.to(device), seq_adv.to(device), mask.to(device), **kw)
    c_o = cur.clone().requires_grad_()
    out_o = o.gspo(c_o, old, seq_adv, mask, **kw)
    rtol, atol = (1e-12, 1e-14) if dtype == torch.float64 else (F32_RTOL, 1e-7)
    _check_scalars(out_h, out_o, ["loss", "sequence_ratio_divergence", "sequence_clip_fraction",
                                  "mean_sequence_ratio", "sequence_ratios"], rtol, atol)
    w = torch.randn(cur.shape[0], generator=_gen(3), dtype=dtype)
    (out_h.loss + (out_h.sequence_ratios * w.to(device)).sum() + out_h.mean_sequence_ratio
     + out_h.sequence_ratio_divergence).backward()
    (out_o["loss"] + (out_o["sequence_ratios"] * w).sum() + out_o["mean_sequence_ratio"]
     + out_o["sequence_ratio_divergence"]).backward()
    _close(c_h.grad, c_o.grad, rtol, atol, "grad")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_gspo_token_parity(device, dtype):
    cur, old, adv, mask = _policy_inputs(15, dtype=dtype)
    cur[1, 0] = old[1, 0] + 0.01
    kw = dict(clip_low=3e-4, clip_high=4e-4)
    c_h, out_h, c_o, out_o = _run_both(R.gspo_token_policy_loss, o.gspo_token, cur, old, adv,
                                       mask, device, None, **kw)
    rtol, atol = (1e-12, 1e-14) if dtype == torch.float64 else (F32_RTOL, 1e-7)
    _check_scalars(out_h, out_o, ["loss", "sequence_ratio_divergence", "sequence_clip_fraction",
                                  "mean_sequence_ratio", "sequence_ratios"], rtol, atol)
    (out_h.loss + out_h.mean_sequence_ratio).backward()
    (out_o["loss"] + out_o["mean_sequence_ratio"]).backward()
    _close(c_h.grad, c_o.grad, rtol, atol, "grad")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("taus", [(1.0, 1.05), (1.0, 1.0), (0.5, 3.0)])
def test_sapo_parity(device, dtype, taus):
    cur, old, adv, mask = _policy_inputs(16, dtype=dtype)
    kw = dict(tau_positive=taus[0], tau_negative=taus[1])
    c_h, out_h, c_o, out_o = _run_both(R.sapo_policy_loss, o.sapo, cur, old, adv, mask, device,
                                       None, **kw)
    rtol, atol = (1e-12, 1e-14) if dtype == torch.float64 else (F32_RTOL, 1e-7)
    _check_scalars(out_h, out_o, ["loss", "approximate_kl", "mean_ratio", "mean_gradient_gate"],
                   rtol, atol)
    (out_h.loss + out_h.approximate_kl + 2 * out_h.mean_ratio - out_h.mean_gradient_gate).backward()
    (out_o["loss"] + out_o["approximate_kl"] + 2 * out_o["mean_ratio"]
     - out_o["mean_gradient_gate"]).backward()
    _close(c_h.grad, c_o.grad, rtol, atol, "grad")


def test_bf16_logprob_inputs_within_2e3(device):
    """Objectives on bf16 log-probs: within 2e-3 of the fp32-upcast oracle."""

    cur, old, adv, mask = _policy_inputs(17)
    cb, ob, ab = cur.bfloat16(), old.bfloat16(), adv.bfloat16()
    out_h = R.clipped_policy_loss(cb.to(device), ob.to(device), ab.to(device), mask.to(device))
    out_o = o.ppo_clip(cb.float(), ob.float(), ab.float(), mask)
    _close(out_h.loss.float(), out_o["loss"], 2e-3, 1e-4, "bf16 loss")


def test_sequence_log_ratio_and_masked_mean(device):
    cur, old, _, mask = _policy_inputs(18)
    c_h = cur.to(device).requires_grad_()
    for norm in (True, False):
        got = L.sequence_log_ratio(c_h, old.to(device), mask.to(device), length_normalize=norm)
        want = o.sequence_log_ratio(cur, old, mask, length_normalize=norm)
        _close(got, want, F32_RTOL, 1e-6, f"seq log ratio norm={norm}")
    v = torch.randn(5, 7, generator=_gen(4))
    wm = torch.rand(5, 7, generator=_gen(5))
    v_h = v.to(device).requires_grad_()
    got = L.masked_mean(v_h, wm.to(device))
    v_o = v.clone().requires_grad_()
    want = o.weighted_average(v_o, wm)
    _close(got, want, F32_RTOL, 1e-7, "masked_mean")
    got.backward()
    want.backward()
    _close(v_h.grad, v_o.grad, F32_RTOL, 1e-8, "masked_mean grad")
    with pytest.raises(ValueError, match="empty mask"):
        L.masked_mean(v.to(device), torch.zeros(5, 7, device=device))
    with pytest.raises(ValueError, match="every sequence"):
        m2 = mask.clone()
        m2[3] = False
        L.sequence_log_ratio(cur.to(device), old.to(device), m2.to(device))


def test_per_row_objectives_reject_empty_rows(device):
    cur, old, adv, mask = _policy_inputs(19)
    mask[2] = False
    d = lambda t: t.to(device)
    with pytest.raises(ValueError, match="every sequence"):
        R.sapo_policy_loss(d(cur), d(old), d(adv), d(mask))
    with pytest.raises(ValueError, match="every sequence"):
        R.gspo_policy_loss(d(cur), d(old), d(adv[:, 0]), d(mask), clip_low=0.1, clip_high=0.1)
    with pytest.raises(ValueError, match="empty mask"):
        R.sao_policy_loss(d(cur), d(old), d(adv), d(torch.zeros_like(mask)), clip_low=0.2,
                          clip_high=0.2)


def test_direct_double_sided_mask_dtypes(device):
    for dt in (torch.float32, torch.float64, torch.bfloat16):
        r = torch.tensor([0.8, 0.800001, 1.0, 1.199999, 1.2, 0.79, 1.21], dtype=dt)
        got = R.direct_double_sided_mask(r.to(device), clip_low=0.2, clip_high=0.2).cpu()
        want = o.strict_trust(r, clip_low=0.2, clip_high=0.2)
        assert torch.equal(got, want), (dt, got, want)


# ---------------------------------------------------------------------------
# estimators
# ---------------------------------------------------------------------------


def _est_inputs(seed, B, T, dtype=torch.float32):
    g = _gen(seed)
    r = torch.randn(B, T, generator=g, dtype=torch.float64).to(dtype)
    v = (torch.randn(B, T, generator=g, dtype=torch.float64) * 0.5).to(dtype)
    valid = torch.rand(B, T, generator=g) < 0.85
    term = torch.rand(B, T, generator=g) < 0.02
    boot = torch.randn(B, generator=g, dtype=torch.float64).to(dtype)
    return r, v, valid, term, boot


def _scale_tol(want, rtol):
    return rtol * max(1.0, want.abs().max().item())


@pytest.mark.parametrize("B,T", [(3, 17), (4, 1000), (2, 8192)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_returns_and_gae_parity(device, B, T, dtype):
    print(f"[estimators] B={B} T={T} dtype={dtype}", flush=True)
    r, v, valid, term, boot = _est_inputs(B * T, B, T, dtype)
    d = lambda t: t.to(device)
    rtol = 1e-12 if dtype == torch.float64 else F32_RTOL
    got = R.discounted_returns(d(r), gamma=0.99, terminated=d(term), valid_mask=d(valid),
                               bootstrap_value=d(boot))
    want = o.returns_to_go(r, gamma=0.99, terminated=term, valid_mask=valid, bootstrap_value=boot)
    _close(got, want, rtol, _scale_tol(want, rtol), "returns")
    for gamma, lam in ((1.0, 0.95), (0.9, 1.0), (0.97, 0.0)):
        ga, gt = R.generalized_advantage_estimation(d(r), d(v), gamma=gamma, gae_lambda=lam,
                                                    terminated=d(term), valid_mask=d(valid),
                                                    bootstrap_value=d(boot))
        wa, wt = o.gae(r, v, gamma=gamma, gae_lambda=lam, terminated=term, valid_mask=valid,
                       bootstrap_value=boot)
        _close(ga, wa, rtol, _scale_tol(wa, rtol), f"gae adv {gamma},{lam}")
        _close(gt, wt, rtol, _scale_tol(wt, rtol), f"gae targets {gamma},{lam}")
    e, n = v, torch.roll(v, -1, dims=-1)
    ga, gt = R.skip_observation_generalized_advantage_estimation(
        d(r), d(e), d(n), gamma=0.95, gae_lambda=0.9, terminated=d(term), valid_mask=d(valid))
    wa, wt = o.skip_observation_gae(r, e, n, gamma=0.95, gae_lambda=0.9, terminated=term,
                                    valid_mask=valid)
    _close(ga, wa, rtol, _scale_tol(wa, rtol), "skip-obs adv")
    _close(gt, wt, rtol, _scale_tol(wt, rtol), "skip-obs targets")


def test_estimators_default_masks_and_batch_dims(device):
    g = _gen(21)
    r = torch.randn(2, 3, 50, generator=g)
    v = torch.randn(2, 3, 50, generator=g)
    ga, gt = R.generalized_advantage_estimation(r.to(device), v.to(device), gamma=0.9,
                                                gae_lambda=0.8)
    wa, wt = o.gae(r, v, gamma=0.9, gae_lambda=0.8)
    _close(ga, wa, F32_RTOL, 1e-5, "gae 3-d")
    r1 = torch.randn(37, generator=g)
    _close(R.discounted_returns(r1.to(device), gamma=0.7), o.returns_to_go(r1, gamma=0.7),
           F32_RTOL, 1e-5, "returns 1-d")


def test_group_and_loo_and_broadcast(device):
    g = _gen(22)
    r = torch.randn(32, 8, generator=g)
    r[3] = 1.0
    r[4, :] = torch.tensor([0.0, 1.0] * 4)
    got = R.group_standardized_advantages(r.to(device)).cpu()
    want = o.group_standardize(r)
    _close(got, want, F32_RTOL, 1e-6, "group std")
    assert torch.equal(got[3], torch.zeros(8))
    got = R.group_standardized_advantages(r.t().contiguous().to(device), dim=0).cpu()
    _close(got, o.group_standardize(r.t().contiguous(), dim=0), F32_RTOL, 1e-6, "group std dim0")
    _close(R.leave_one_out_advantages(r.to(device)), o.leave_one_out(r), F32_RTOL, 1e-6, "loo")
    ta = torch.randn(5, 4, generator=g)
    ids = torch.randint(0, 4, (5, 33), generator=g)
    m = torch.rand(5, 33, generator=g) < 0.6
    ids[~m] = -7
    got = R.broadcast_turn_advantages(ta.to(device), ids.to(device), m.to(device)).cpu()
    assert torch.equal(got, o.turn_broadcast(ta, ids, m))
    ids[0, 0], m[0, 0] = 4, True
    with pytest.raises(ValueError, match="invalid turn"):
        R.broadcast_turn_advantages(ta.to(device), ids.to(device), m.to(device))


def test_masked_whiten(device):
    g = _gen(23)
    x = torch.randn(64, 300, generator=g) * 3 + 1
    m = torch.rand(64, 300, generator=g) < 0.5
    got = R.masked_whiten(x.to(device), m.to(device))
    _close(got, o.masked_whiten(x, m), 1e-5, 1e-5, "whiten")
    sel = got.cpu()[m].double()
    assert abs(sel.mean().item()) < 1e-5 and abs(sel.std(unbiased=False).item() - 1) < 1e-5


# ---------------------------------------------------------------------------
# single pass vs composition
# ---------------------------------------------------------------------------


def _fused_inputs(seed, B, T, V, dtype):
    g = _gen(seed)
    x = (torch.randn(B, T, V, generator=g) * 3.0).to(dtype)
    rows = torch.rand(B, T, generator=g) < 0.05
    hot = torch.randint(0, V, (B, T), generator=g)
    xf = x.float()
    xf[rows, hot[rows]] += 15.0
    x = xf.to(dtype)
    probs = torch.softmax(x.float(), dim=-1)
    t = torch.multinomial(probs.reshape(-1, V), 1, generator=g).reshape(B, T)
    lp = o.token_logprobs(x, t)
    old = lp + torch.randn(B, T, generator=g) * 0.1
    lengths = torch.randint(1, T + 1, (B,), generator=g)
    mask = torch.arange(T)[None, :] < lengths[:, None]
    r = torch.randint(0, 2, (B // 4, 4), generator=g).float()
    adv = o.group_standardize(r).reshape(-1)[:, None].expand(B, T)
    return x, t, old, adv, mask


@pytest.mark.parametrize("objective", ["clipped", "sao", "sapo", "gspo", "gspo_token"])
@pytest.mark.parametrize("dtype,V", [(torch.float32, 50257), (torch.bfloat16, 151936)])
def test_fused_matches_oracle(device, objective, dtype, V):
    print(f"[fused] objective={objective} dtype={dtype} V={V}", flush=True)
    B, T = 8, 16
    x, t, old, adv, mask = _fused_inputs(31, B, T, V, dtype)
    kw = {"clipped": dict(clip_low=0.2, clip_high=0.28), "sao": dict(clip_low=0.2, clip_high=0.28),
          "sapo": dict(tau_positive=1.0, tau_negative=1.05),
          "gspo": dict(clip_low=3e-4, clip_high=4e-4),
          "gspo_token": dict(clip_low=3e-4, clip_high=4e-4)}[objective]
    a = adv[:, 0].contiguous() if objective == "gspo" else adv
    xd = x.to(device).requires_grad_()
    out, lp = R.fused_policy_loss(xd, t.to(device), old.to(device), a.to(device),
                                  mask.to(device), objective=objective, return_logprobs=True,
                                  **kw)
    out.loss.backward()
    kind = {"clipped": "ppo"}.get(objective, objective)
    out_o, lpo, dlo = o.policy_step(kind, x, t, old, a, mask, exact=True, **kw)
    _close(lp, lpo, F32_RTOL, 1e-7, "logp")
    # The loss is a signed sum of per-token terms of size ~|A| that largely
    # cancel (group-standardized A has mean 0), so its relative tolerance is
    # taken against the terms' scale, not the near-zero sum.
    scale = max(abs(out_o["loss"].item()), a.abs().mean().item())
    rt = F32_RTOL if dtype == torch.float32 else 2e-3
    assert abs(out.loss.item() - out_o["loss"].item()) <= rt * scale, (
        out.loss.item(), out_o["loss"].item())
    if dtype == torch.float32:
        _close_rows_by_g(xd.grad, dlo, out_o["dloss_dlogp"], F32_RTOL, "dlogits")
    else:
        assert _ulp16(xd.grad, dlo, "dlogits") > 0.98
        _rownorm16(xd.grad, dlo, 2e-3, "dlogits")


def test_fused_equals_composition_and_grad_scaling(device):
    B, T, V = 4, 8, 3001
    x, t, old, adv, mask = _fused_inputs(32, B, T, V, torch.float32)
    d = lambda z: z.to(device)
    x1 = d(x).requires_grad_()
    out1 = R.fused_policy_loss(x1, d(t), d(old), d(adv), d(mask), clip_low=0.2, clip_high=0.28)
    (3.0 * out1.loss).backward()
    x2 = d(x).requires_grad_()
    lp2 = R.gather_token_logprobs(x2, d(t))
    out2 = R.clipped_policy_loss(lp2, d(old), d(adv), d(mask), clip_low=0.2, clip_high=0.28)
    (3.0 * out2.loss).backward()
    _close(out1.loss, out2.loss, 1e-6, 1e-8, "loss")
    _close(x1.grad, x2.grad, 1e-5, 1e-9, "scaled dlogits")
    # diagnostics receive gradient too: general backward path
    x3 = d(x).requires_grad_()
    out3 = R.fused_policy_loss(x3, d(t), d(old), d(adv), d(mask), clip_low=0.2, clip_high=0.28)
    (out3.loss + 0.5 * out3.approximate_kl).backward()
    x4 = d(x).requires_grad_()
    lp4 = R.gather_token_logprobs(x4, d(t))
    out4 = R.clipped_policy_loss(lp4, d(old), d(adv), d(mask), clip_low=0.2, clip_high=0.28)
    (out4.loss + 0.5 * out4.approximate_kl).backward()
    _close(x3.grad, x4.grad, 1e-5, 1e-9, "dlogits with kl term")


def test_fused_inplace(device):
    B, T, V = 4, 8, 4096
    x, t, old, adv, mask = _fused_inputs(33, B, T, V, torch.bfloat16)
    d = lambda z: z.to(device)
    ref = d(x).requires_grad_()
    out_r = R.fused_policy_loss(ref, d(t), d(old), d(adv), d(mask), objective="sapo")
    out_r.loss.backward()
    buf = d(x).detach()
    out_i = R.fused_policy_loss(buf.requires_grad_(), d(t), d(old), d(adv), d(mask),
                                objective="sapo", inplace=True)
    _close(out_i.loss, out_r.loss, 1e-6, 1e-8, "inplace loss")
    assert torch.equal(buf.detach().cpu(), ref.grad.cpu()), "in-place dlogits differ"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("objective", ["clipped", "sao", "sapo"])
def test_fused_many_rows_persistent(device, dtype, objective):
    """More rows than workgroups: every workgroup carries several rows and
    prefetches the next one into its registers (16-bit resident path).  V =
    20000 leaves the last register slab of each row partially filled."""

    print(f"[fused-many] objective={objective} dtype={dtype}", flush=True)
    B, T, V = 64, 40, 20000
    x, t, old, adv, mask = _fused_inputs(34, B, T, V, dtype)
    kw = {"clipped": dict(clip_low=0.2, clip_high=0.28),
          "sao": dict(clip_low=0.2, clip_high=0.28),
          "sapo": dict(tau_positive=1.0, tau_negative=1.05)}[objective]
    xd = x.to(device).requires_grad_()
    out, lp = R.fused_policy_loss(xd, t.to(device), old.to(device), adv.to(device),
                                  mask.to(device), objective=objective, return_logprobs=True,
                                  **kw)
    out.loss.backward()
    kind = {"clipped": "ppo"}.get(objective, objective)
    out_o, lpo, dlo = o.policy_step(kind, x, t, old, adv, mask, exact=True, **kw)
    _close(lp, lpo, F32_RTOL, 1e-7, "logp")
    scale = max(abs(out_o["loss"].item()), adv.abs().mean().item())
    assert abs(out.loss.item() - out_o["loss"].item()) <= 2e-3 * scale
    assert _ulp16(xd.grad, dlo, "dlogits") > 0.98
    _rownorm16(xd.grad, dlo, 2e-3, "dlogits")
    # masked rows carry exactly zero gradient
    assert torch.count_nonzero(xd.grad[~mask.to(device)]).item() == 0


def test_fused_extreme_logits(device):
    """Rows at the edge of the 16-bit range: an all -inf row but one entry, a
    half -inf (masked vocabulary) row, and a row whose log-sum-exp (3e38)
    exceeds the register-resident kernel's exponent range, which the generic
    kernel launched behind it (RRL_POLICY_RERUN_FAST_RANGE) then redoes on the
    device.  All must match the float64 oracle."""

    B, T, V = 4, 8, 4096
    x, t, old, adv, mask = _fused_inputs(35, B, T, V, torch.bfloat16)
    xf = x.float()
    xf[0, 1, :] = -float("inf")
    xf[0, 1, 5] = 0.0
    t[0, 1] = 5
    xf[0, 2, : V // 2] = -float("inf")
    t[0, 2] = V - 3
    xf[1, 3, 7] = 3.0e38
    t[1, 3] = 7
    xf[1, 4, 9] = 3.0e38
    t[1, 4] = 11  # log-prob of about -3e38: the ratio clamps at max_log_ratio
    x = xf.to(torch.bfloat16)
    mask[:, :6] = True
    old = o.token_logprobs(x, t, exact=True).float() + 0.05
    old[1, 4] = -5.0
    kw = dict(clip_low=0.2, clip_high=0.28)
    xd = x.to(device).requires_grad_()
    out, lp = R.fused_policy_loss(xd, t.to(device), old.to(device), adv.to(device),
                                  mask.to(device), return_logprobs=True, **kw)
    out.loss.backward()
    out_o, lpo, dlo = o.policy_step("ppo", x, t, old, adv, mask, exact=True, **kw)
    _close(lp, lpo, F32_RTOL, 1e-7, "logp")
    scale = max(abs(out_o["loss"].item()), adv.abs().mean().item())
    assert abs(out.loss.item() - out_o["loss"].item()) <= 2e-3 * scale
    assert _ulp16(xd.grad, dlo, "dlogits") > 0.98
    _rownorm16(xd.grad, dlo, 2e-3, "dlogits")


@pytest.mark.parametrize("V", [4096, 151936])
def test_fused_rerun_only_when_flagged(device, V):
    """The conditional generic launch queued behind an out-of-place bfloat16
    sweep returns at once when no row was flagged: log-probs, loss and
    dlogits equal the register-resident kernel's own (an in-place call, which
    queues no rerun) bit for bit."""

    print(f"[rerun-if-flagged] V={V}", flush=True)
    B, T = 4, 8
    x, t, old, adv, mask = _fused_inputs(73, B, T, V, torch.bfloat16)
    d = lambda v: v.to(device)  # noqa: E731
    kw = dict(clip_low=0.2, clip_high=0.28, return_logprobs=True)
    xd = d(x).requires_grad_()
    out, lp = R.fused_policy_loss(xd, d(t), d(old), d(adv), d(mask), **kw)
    out.loss.backward()
    buf = d(x).detach()
    out_i, lp_i = R.fused_policy_loss(buf.requires_grad_(), d(t), d(old), d(adv), d(mask),
                                      inplace=True, **kw)
    assert torch.equal(lp, lp_i)
    _close(out_i.loss, out.loss, 1e-6, 1e-8, "loss")
    assert torch.equal(buf.detach(), xd.grad), "dlogits differ from the resident kernel's"


@pytest.mark.parametrize("dtype,V", [(torch.bfloat16, 151936), (torch.bfloat16, 20000),
                                     (torch.float32, 3001)])
@pytest.mark.parametrize("objective", ["clipped", "sapo"])
def test_fused_skip_masked_rows_bit_identical(device, dtype, V, objective):
    """skip_masked_rows=True never reads zero-weight rows; for finite logits the
    loss, diagnostics and dlogits equal the default path bit for bit."""

    print(f"[skip-masked] objective={objective} dtype={dtype} V={V}", flush=True)
    B, T = 16, 24
    x, t, old, adv, mask = _fused_inputs(37, B, T, V, dtype)
    kw = {"clipped": dict(clip_low=0.2, clip_high=0.28),
          "sapo": dict(tau_positive=1.0, tau_negative=1.05)}[objective]
    d = lambda z: z.to(device)
    outs, grads = [], []
    for skip in (False, True):
        xd = d(x).requires_grad_()
        out = R.fused_policy_loss(xd, d(t), d(old), d(adv), d(mask), objective=objective,
                                  skip_masked_rows=skip, **kw)
        out.loss.backward()
        outs.append(out)
        grads.append(xd.grad)
    for f in ("loss", "approximate_kl", "mean_ratio"):
        assert torch.equal(getattr(outs[0], f), getattr(outs[1], f)), f
    assert torch.equal(grads[0], grads[1])
    assert torch.count_nonzero(grads[1][~d(mask)]).item() == 0
    with pytest.raises(ValueError, match="return_logprobs"):
        R.fused_policy_loss(d(x), d(t), d(old), d(adv), d(mask), objective=objective,
                            skip_masked_rows=True, return_logprobs=True, **kw)


@pytest.mark.parametrize("dtype,V", [(torch.bfloat16, 151936), (torch.float32, 3001),
                                     (torch.float16, 4099)])
@pytest.mark.parametrize("objective", ["gspo", "gspo_token"])
def test_gspo_skip_masked_rows_bit_identical(device, dtype, V, objective):
    """GSPO's forward sweep with skip_masked_rows=True does not read masked
    tokens (their log-probs enter the sequence log-ratio only times their zero
    mask): loss, diagnostics and dlogits equal the default bit for bit, masked
    dlogits rows are zero, and a NaN logit at a masked position no longer
    reaches the loss (the default, like the reference's 0 * NaN, gives NaN)."""

    print(f"[gspo-skip] objective={objective} dtype={dtype} V={V}", flush=True)
    B, T = 16, 24
    x, t, old, adv, mask = _fused_inputs(38, B, T, V, dtype)
    a = adv[:, 0].contiguous() if objective == "gspo" else adv
    kw = dict(clip_low=3e-4, clip_high=4e-4)
    d = lambda z: z.to(device)  # noqa: E731
    outs, grads = [], []
    for skip in (False, True):
        xd = d(x).requires_grad_()
        out = R.fused_policy_loss(xd, d(t), d(old), d(a), d(mask), objective=objective,
                                  skip_masked_rows=skip, **kw)
        out.loss.backward()
        outs.append(out)
        grads.append(xd.grad)
    fields = [f for f in ("loss", "objective", "sequence_ratio_divergence",
                          "sequence_clip_fraction", "mean_sequence_ratio", "sequence_ratios",
                          "approximate_kl", "mean_ratio") if hasattr(outs[0], f)]
    assert fields
    for f in fields:
        assert torch.equal(getattr(outs[0], f), getattr(outs[1], f)), f
    assert torch.equal(grads[0], grads[1])
    assert torch.count_nonzero(grads[1][~d(mask)]).item() == 0
    # a NaN logit at a masked token: read (and propagated) only by the default
    xn = x.clone()
    b, tt = torch.nonzero(~mask)[0].tolist()
    xn[b, tt, 0] = float("nan")
    ln = R.fused_policy_loss(d(xn), d(t), d(old), d(a), d(mask), objective=objective,
                             skip_masked_rows=True, **kw).loss
    assert torch.equal(ln, outs[1].loss)
    l0 = R.fused_policy_loss(d(xn), d(t), d(old), d(a), d(mask), objective=objective, **kw).loss
    assert torch.isnan(l0)


@pytest.mark.parametrize(
    "dtype,V,B,T",
    [
        (torch.float32, 50257, 4, 68),  # config 1's vocabulary, 272 rows: every head offset
        (torch.float32, 81923, 4, 1),  # 20 slabs of float32 vectors
        (torch.float32, 7, 4, 5),  # head and tail elements only
        (torch.float32, 1, 4, 5),  # the target is the row's only element, a head or tail one
        (torch.bfloat16, 1, 4, 5),
        (torch.bfloat16, 50257, 4, 68),
        (torch.float16, 4099, 4, 7),
        (torch.bfloat16, 163843, 4, 1),  # 20 full slabs and a tail
        (torch.bfloat16, 3, 4, 3),
    ],
)
@pytest.mark.parametrize("objective", ["clipped", "sapo"])
def test_fused_resident_head_tail_rows(device, dtype, V, B, T, objective):
    """Rows that do not start on a 16-byte boundary or whose length is not a
    whole number of 16-byte vectors: the register-resident kernel carries the
    head and tail elements beside its aligned slabs.  Held against the
    float64 oracle and against the generic row kernel, reached through a
    logits view whose rows sit at a different offset from the dlogits rows."""

    print(f"[fused-headtail] objective={objective} dtype={dtype} V={V} B={B} T={T}", flush=True)
    x, t, old, adv, mask = _fused_inputs(40 + V % 97, B, T, V, dtype)
    kw = (dict(clip_low=0.2, clip_high=0.28) if objective == "clipped"
          else dict(tau_positive=1.0, tau_negative=1.05))
    d = lambda z: z.to(device)  # noqa: E731
    xd = d(x).requires_grad_()
    out, lp = R.fused_policy_loss(xd, d(t), d(old), d(adv), d(mask), objective=objective,
                                  return_logprobs=True, **kw)
    out.loss.backward()
    kind = {"clipped": "ppo"}.get(objective, objective)
    out_o, lpo, dlo = o.policy_step(kind, x, t, old, adv, mask, exact=True, **kw)
    _close(lp, lpo, F32_RTOL, 1e-7, "logp")
    scale = max(abs(out_o["loss"].item()), adv.abs().mean().item())
    rt = F32_RTOL if dtype == torch.float32 else 2e-3
    assert abs(out.loss.item() - out_o["loss"].item()) <= rt * scale
    if dtype == torch.float32:
        _close_rows_by_g(xd.grad, dlo, out_o["dloss_dlogp"], F32_RTOL, "dlogits")
    else:
        assert _ulp16(xd.grad, dlo, "dlogits") > 0.98
        _rownorm16(xd.grad, dlo, 2e-3, "dlogits")
    # generic kernel: logits rows one element off the dlogits rows' offset
    wide = torch.empty(B, T, V + 1, dtype=dtype, device=device)
    wide[..., 1:] = d(x)
    xg = wide[..., 1:].requires_grad_()
    out_g, lp_g = R.fused_policy_loss(xg, d(t), d(old), d(adv), d(mask), objective=objective,
                                      return_logprobs=True, **kw)
    out_g.loss.backward()
    _close(lp, lp_g, F32_RTOL, 1e-7, "logp resident vs generic")
    if dtype == torch.float32:
        _close_rows_by_g(xd.grad, xg.grad, out_o["dloss_dlogp"], F32_RTOL, "resident vs generic")
    else:
        _ulp16(xd.grad, xg.grad.float(), "resident vs generic")
