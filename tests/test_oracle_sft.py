"""The SFT cross-entropy oracle (rosetrainer/model.py:643-649) pinned on the
CPU: against torch's own F.cross_entropy in float64 (the library routine the
reference calls), against the scalar loops of oracle/brute.py, and against
closed forms; planted mistakes in the restatement must fail these pins.  Also
the Python API's argument checks, which run before any device work."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import brute
from oracle import roserlhf_oracle as o


def _case(seed, N=40, V=37, ignore=-100, frac_ignored=0.25):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, V, generator=g, dtype=torch.float64) * 2.5
    y = torch.randint(0, V, (N,), generator=g)
    drop = torch.rand(N, generator=g) < frac_ignored
    y[drop] = ignore
    return x, y


@pytest.mark.parametrize("reduction", ["mean", "sum"])
@pytest.mark.parametrize("ignore", [-100, 3])
def test_nll_matches_torch_cross_entropy(reduction, ignore):
    x, y = _case(1 + (ignore > 0), ignore=ignore)
    xa = x.clone().requires_grad_()
    loss = o.nll_loss(xa, y, ignore_index=ignore, reduction=reduction)
    loss.backward()
    xb = x.clone().requires_grad_()
    want = F.cross_entropy(xb, y, ignore_index=ignore, reduction=reduction)
    want.backward()
    assert abs(loss.item() - want.item()) <= 1e-12 * abs(want.item())
    assert torch.allclose(xa.grad, xb.grad, rtol=1e-12, atol=1e-15)


def test_causal_step_matches_model_forward_expression():
    g = torch.Generator().manual_seed(5)
    B, T, V = 3, 9, 23
    logits = torch.randn(B, T, V, generator=g, dtype=torch.float64) * 3
    labels = torch.randint(0, V, (B, T), generator=g)
    labels[0, 4] = -100
    loss, dl = o.sft_step(logits, labels, causal=True)
    # rosetrainer/model.py:644-649, verbatim semantics
    x = logits.clone().requires_grad_()
    shift_logits = x[:, :-1, :].contiguous()
    shift_labels = labels[:, 1:].contiguous()
    want = F.cross_entropy(shift_logits.view(-1, V), shift_labels.view(-1))
    want.backward()
    assert abs(loss.item() - want.item()) <= 1e-12 * abs(want.item())
    assert torch.allclose(dl, x.grad, rtol=1e-12, atol=1e-15)
    assert (dl[:, -1] == 0).all()


@pytest.mark.parametrize("reduction", ["mean", "sum"])
def test_nll_matches_brute_force(reduction):
    x, y = _case(7, N=12, V=11)
    loss, dl = o.sft_step(x, y, causal=False, reduction=reduction, exact=True)
    want = brute.nll_loss(x.numpy(), y.numpy(), reduction=reduction)
    assert abs(loss.item() - want) <= 1e-12 * abs(want)
    g = brute.nll_grad(y.numpy(), reduction=reduction)
    safe = np.where(y.numpy() == -100, 0, y.numpy())
    want_dl = brute.dlogits_from_g(x.numpy(), safe, -g)
    # loss = -objective: dlogits = -(d objective / d logits) = g_loss * (softmax - onehot)
    np.testing.assert_allclose(dl.numpy(), -want_dl, rtol=1e-10, atol=1e-14)


def test_known_answers():
    V = 50
    # Uniform logits: every label has log p = -log V.
    x = torch.zeros(6, V, dtype=torch.float64)
    y = torch.tensor([0, 5, 49, -100, 7, 7])
    assert abs(o.nll_loss(x, y).item() - math.log(V)) < 1e-14
    assert abs(o.nll_loss(x, y, reduction="sum").item() - 5 * math.log(V)) < 1e-12
    # All ignored: NaN mean and zero gradients (F.cross_entropy's behaviour).
    loss, dl = o.sft_step(x, torch.full((6,), -100), causal=False)
    assert math.isnan(loss.item()) and (dl == 0).all()
    # Dominant label: loss -> log(1 + (V-1) e^-30).
    x2 = torch.zeros(1, V, dtype=torch.float64)
    x2[0, 3] = 30.0
    assert abs(o.nll_loss(x2, torch.tensor([3])).item() - math.log1p((V - 1) * math.exp(-30))) < 1e-14


def test_range_errors():
    x = torch.zeros(3, 5, dtype=torch.float64)
    with pytest.raises(IndexError):
        o.nll_loss(x, torch.tensor([1, 5, 2]))
    with pytest.raises(IndexError):
        o.nll_loss(x, torch.tensor([1, -7, 2]))
    # ignore_index is never range-checked; with another ignore_index -100 is
    with pytest.raises(IndexError):
        o.nll_loss(x, torch.tensor([1, -100, 2]), ignore_index=2)
    assert math.isfinite(o.nll_loss(x, torch.tensor([1, -100, 2])).item())


def _mean_over_all_tokens(logits, labels, *, ignore_index=-100, reduction="mean", exact=False):
    keep = labels.reshape(-1) != ignore_index
    lp = o.token_logprobs(logits.reshape(-1, logits.shape[-1]),
                          torch.where(keep, labels.reshape(-1), 0))
    return -(torch.where(keep, lp, torch.zeros_like(lp)).sum() / keep.numel())


def _ignored_gathered_at_zero(logits, labels, *, ignore_index=-100, reduction="mean", exact=False):
    keep = labels.reshape(-1) != ignore_index
    lp = o.token_logprobs(logits.reshape(-1, logits.shape[-1]),
                          torch.where(keep, labels.reshape(-1), 0))
    return -(lp.sum() / keep.sum())


@pytest.mark.parametrize("planted", [_mean_over_all_tokens, _ignored_gathered_at_zero])
def test_planted_mistakes_fail_the_pins(planted, monkeypatch):
    x, y = _case(11)
    monkeypatch.setattr(o, "nll_loss", planted)
    got = o.nll_loss(x, y).item()
    want = F.cross_entropy(x, y).item()
    assert abs(got - want) > 1e-6 * abs(want)
    assert abs(got - brute.nll_loss(x.numpy(), y.numpy())) > 1e-6 * abs(want)


# ---------------------------------------------------------------------------
# API checks that run before any device work (no GPU needed)
# ---------------------------------------------------------------------------


def test_api_argument_checks():
    from rosellm_amd import rosetrainer as RT

    x = torch.zeros(4, 7)
    with pytest.raises(ValueError, match="batch_size"):
        RT.cross_entropy(x, torch.zeros(3, dtype=torch.long))
    with pytest.raises(RuntimeError, match="expected scalar type Long"):
        RT.cross_entropy(x, torch.zeros(4))
    with pytest.raises(ValueError, match="not a valid value for reduction"):
        RT.cross_entropy(x, torch.zeros(4, dtype=torch.long), reduction="avg")
    with pytest.raises(ValueError, match="reduction='none'"):
        RT.cross_entropy(x, torch.zeros(4, dtype=torch.long), reduction="none")
    with pytest.raises(ValueError, match="class dimension"):
        RT.cross_entropy(torch.zeros(4), torch.zeros((), dtype=torch.long))
    with pytest.raises(ValueError, match="batch, positions"):
        RT.causal_lm_loss(x, torch.zeros(4, dtype=torch.long))
    with pytest.raises(ValueError, match="must match logits prefix"):
        RT.causal_lm_loss(torch.zeros(2, 3, 5), torch.zeros(2, 4, dtype=torch.long))
    # Valid arguments on the CPU: the package has no CPU path and says so.
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        RT.cross_entropy(x, torch.zeros(4, dtype=torch.long))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        RT.linear_causal_lm_loss(torch.zeros(2, 3, 4), torch.zeros(5, 4),
                                 torch.zeros(2, 3, dtype=torch.long))
