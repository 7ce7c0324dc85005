"""Pin the CPU oracle (oracle/roserlhf_oracle.py) before trusting it.

Four independent checks, each chosen so a plausible slip in the restatement
(dropped term, wrong sign or index, wrong tie/boundary rule) fails one:
  1. every transcribed reference known answer (tests/golden/known_answers.json);
  2. float64 scalar-loop brute force written from the definitions (oracle/brute.py);
  3. closed-form d loss / d logp per objective vs the oracle's autograd;
  4. reference invariants (padding invariance, GSPO == GSPO-token for uniform
     advantages, GAE(lambda=1) == Monte-Carlo return - V, ...).
Plus planted mistakes: mutated oracle variants must fail these pins.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import brute
from oracle import roserlhf_oracle as o
from tests._cases import CASE_IDS, CASES, run_case


@pytest.mark.parametrize("case", CASES, ids=CASE_IDS)
def test_known_answer_oracle(case):
    run_case(case, "oracle", "cpu")


def _rng(seed=0):
    return np.random.default_rng(seed)


def test_logprob_vs_brute_force():
    rng = _rng(1)
    x = rng.normal(0, 3.0, size=(3, 5, 37))
    x[0, 0, 3] += 15.0  # dominant logit
    x[1, 2, :5] = -np.inf  # masked vocabulary entries
    t = rng.integers(5, 37, size=(3, 5))
    t[0, 0] = 3
    got = o.token_logprobs(torch.tensor(x), torch.tensor(t)).numpy()
    want = brute.logprob(np.where(np.isinf(x), -1e300, x), t)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_logprob_bf16_is_fp32_upcast():
    rng = _rng(2)
    x = torch.tensor(rng.normal(0, 3.0, size=(4, 50)), dtype=torch.bfloat16)
    t = torch.tensor(rng.integers(0, 50, size=(4,)))
    got = o.token_logprobs(x, t)
    assert got.dtype == torch.float32
    want = brute.logprob(x.float().double().numpy(), t.numpy())
    np.testing.assert_allclose(got.numpy(), want, rtol=2e-6, atol=2e-6)


def _planted_inputs(rng, B=4, T=9, lo=0.8, hi=1.2, K=20.0):
    """Random log-probs with ties and boundaries planted on purpose."""

    old = rng.normal(-2.0, 1.0, size=(B, T))
    cur = old + rng.normal(0, 0.3, size=(B, T))
    cur[0, 0] = old[0, 0] + math.log(lo)  # ratio exactly at the lower bound
    cur[0, 1] = old[0, 1] + math.log(hi)  # ... and at the upper bound
    cur[1, 0] = old[1, 0] + K  # log-ratio exactly at the clamp bound
    cur[1, 1] = old[1, 1] + K + 3.0  # beyond the clamp
    adv = rng.normal(0, 1, size=(B, T))
    adv[2, :3] = 0.0  # zero advantage ties
    mask = rng.random((B, T)) < 0.8
    mask[:, 0] = True
    return cur, old, adv, mask


def _oracle_grad(fn, cur, *rest, **kw):
    c = torch.tensor(cur, requires_grad=True)
    args = [torch.tensor(a) if not isinstance(a, torch.Tensor) else a for a in rest]
    out = fn(c, *args, **kw)
    out["objective"].backward()
    return out["objective"].item(), c.grad.numpy()


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_ppo_closed_form(seed):
    rng = _rng(seed)
    cur, old, adv, mask = _planted_inputs(rng)
    w = mask.astype(np.float64)
    obj, g = _oracle_grad(o.ppo_clip, cur, old, adv, torch.tensor(w), clip_low=0.2, clip_high=0.2)
    bobj, bg = brute.ppo_objective_grad(cur, old, adv, w, clip_low=0.2, clip_high=0.2)
    assert obj == pytest.approx(bobj, rel=1e-12, abs=1e-12)
    np.testing.assert_allclose(g.reshape(-1), bg, rtol=1e-12, atol=1e-15)


@pytest.mark.parametrize("detach", [True, False])
def test_sao_closed_form(detach):
    rng = _rng(5)
    cur, old, adv, mask = _planted_inputs(rng)
    obj, g = _oracle_grad(o.sao, cur, old, adv, torch.tensor(mask), clip_low=0.2, clip_high=0.2,
                          detach_ratio=detach)
    bobj, bg = brute.sao_objective_grad(cur, old, adv, mask, clip_low=0.2, clip_high=0.2,
                                        detach=detach)
    assert obj == pytest.approx(bobj, rel=1e-12, abs=1e-12)
    np.testing.assert_allclose(g.reshape(-1), bg, rtol=1e-12, atol=1e-15)


def test_gspo_closed_form():
    rng = _rng(6)
    cur, old, _, mask = _planted_inputs(rng)
    A = rng.normal(0, 1, size=cur.shape[0])
    obj, g = _oracle_grad(o.gspo, cur, old, A, torch.tensor(mask), clip_low=0.05, clip_high=0.08)
    bobj, bg = brute.gspo_objective_grad(cur, old, A, mask, clip_low=0.05, clip_high=0.08)
    assert obj == pytest.approx(bobj, rel=1e-12, abs=1e-12)
    np.testing.assert_allclose(g, bg, rtol=1e-12, atol=1e-15)


def test_gspo_token_closed_form():
    rng = _rng(7)
    cur, old, adv, mask = _planted_inputs(rng)
    obj, g = _oracle_grad(o.gspo_token, cur, old, adv, torch.tensor(mask), clip_low=0.05,
                          clip_high=0.08)
    bobj, bg = brute.gspo_token_objective_grad(cur, old, adv, mask, clip_low=0.05,
                                               clip_high=0.08)
    assert obj == pytest.approx(bobj, rel=1e-12, abs=1e-12)
    np.testing.assert_allclose(g, bg, rtol=1e-12, atol=1e-15)


def test_sapo_closed_form():
    rng = _rng(8)
    cur, old, adv, mask = _planted_inputs(rng)
    obj, g = _oracle_grad(o.sapo, cur, old, adv, torch.tensor(mask), tau_positive=1.0,
                          tau_negative=1.05)
    bobj, bg = brute.sapo_objective_grad(cur, old, adv, mask, tau_positive=1.0,
                                         tau_negative=1.05)
    assert obj == pytest.approx(bobj, rel=1e-12, abs=1e-12)
    np.testing.assert_allclose(g, bg, rtol=1e-12, atol=1e-15)


def test_dlogits_composition_closed_form():
    """Oracle autograd through log-softmax+gather+clip equals g*(onehot - softmax)."""

    rng = _rng(9)
    B, T, V = 2, 6, 23
    x = rng.normal(0, 2.0, size=(B, T, V))
    tgt = rng.integers(0, V, size=(B, T))
    lp = brute.logprob(x, tgt)
    old = lp + rng.normal(0, 0.1, size=lp.shape)
    adv = rng.normal(0, 1, size=lp.shape)
    mask = rng.random(lp.shape) < 0.7
    mask[0, 0] = True
    out, olp, dl = o.grpo_step(torch.tensor(x), torch.tensor(tgt), torch.tensor(old),
                               torch.tensor(adv), torch.tensor(mask), clip_low=0.2,
                               clip_high=0.28)
    np.testing.assert_allclose(olp.numpy(), lp, rtol=1e-12, atol=1e-12)
    _, g_obj = brute.ppo_objective_grad(lp, old, adv, mask.astype(float), clip_low=0.2,
                                        clip_high=0.28)
    want = brute.dlogits_from_g(x, tgt, -g_obj.reshape(B, T))
    np.testing.assert_allclose(dl.numpy(), want, rtol=1e-10, atol=1e-14)


def _masks(rng, shape, p_valid=0.8, p_term=0.1):
    valid = rng.random(shape) < p_valid
    term = rng.random(shape) < p_term
    return valid, term


@pytest.mark.parametrize("seed", [0, 1])
def test_returns_vs_brute(seed):
    rng = _rng(seed)
    r = rng.normal(0, 1, size=(3, 17))
    valid, term = _masks(rng, r.shape)
    boot = rng.normal(0, 1, size=3)
    got = o.returns_to_go(torch.tensor(r), gamma=0.93, terminated=torch.tensor(term),
                          valid_mask=torch.tensor(valid), bootstrap_value=torch.tensor(boot))
    want = brute.returns(r, gamma=0.93, terminated=term, valid=valid, bootstrap=boot)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("seed", [0, 1])
def test_gae_vs_brute(seed):
    rng = _rng(seed + 10)
    r = rng.normal(0, 1, size=(3, 19))
    v = rng.normal(0, 0.5, size=r.shape)
    valid, term = _masks(rng, r.shape)
    boot = rng.normal(0, 1, size=3)
    adv, tgt = o.gae(torch.tensor(r), torch.tensor(v), gamma=0.97, gae_lambda=0.9,
                     terminated=torch.tensor(term), valid_mask=torch.tensor(valid),
                     bootstrap_value=torch.tensor(boot))
    badv, btgt = brute.gae(r, v, gamma=0.97, lam=0.9, terminated=term, valid=valid, bootstrap=boot)
    np.testing.assert_allclose(adv.numpy(), badv, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(tgt.numpy(), btgt, rtol=1e-12, atol=1e-12)


def test_skip_gae_vs_brute():
    rng = _rng(20)
    r = rng.normal(0, 1, size=(2, 11))
    e = rng.normal(0, 1, size=r.shape)
    n = rng.normal(0, 1, size=r.shape)
    valid, term = _masks(rng, r.shape)
    adv, tgt = o.skip_observation_gae(torch.tensor(r), torch.tensor(e), torch.tensor(n),
                                      gamma=0.9, gae_lambda=0.8, terminated=torch.tensor(term),
                                      valid_mask=torch.tensor(valid))
    badv, btgt = brute.skip_gae(r, e, n, gamma=0.9, lam=0.8, terminated=term, valid=valid)
    np.testing.assert_allclose(adv.numpy(), badv, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(tgt.numpy(), btgt, rtol=1e-12, atol=1e-12)


def test_group_loo_broadcast_whiten_vs_brute():
    rng = _rng(30)
    r = rng.normal(0, 1, size=(5, 8))
    r[2] = 0.7  # uniform group -> exactly zero
    np.testing.assert_allclose(o.group_standardize(torch.tensor(r)).numpy(),
                               brute.group_standardize(r), rtol=1e-12, atol=1e-12)
    assert np.all(o.group_standardize(torch.tensor(r)).numpy()[2] == 0.0)
    np.testing.assert_allclose(o.leave_one_out(torch.tensor(r)).numpy(), brute.leave_one_out(r),
                               rtol=1e-12, atol=1e-12)
    ta = rng.normal(0, 1, size=(3, 4))
    ids = rng.integers(0, 4, size=(3, 10))
    m = rng.random((3, 10)) < 0.6
    ids[~m] = 99  # masked positions may carry any id
    assert np.array_equal(o.turn_broadcast(torch.tensor(ta), torch.tensor(ids),
                                           torch.tensor(m)).numpy(),
                          brute.turn_broadcast(ta, np.where(m, ids, 0), m))
    x = rng.normal(0, 2, size=(4, 7))
    wm = rng.random((4, 7)) < 0.5
    wm[0, 0] = True
    np.testing.assert_allclose(o.masked_whiten(torch.tensor(x), torch.tensor(wm)).numpy(),
                               brute.whiten(x, wm), rtol=1e-12, atol=1e-12)


# ---- invariants (reference tests as properties) -----------------------------


def test_gae_lambda_one_equals_mc_minus_value_random():
    rng = _rng(40)
    r = torch.tensor(rng.normal(0, 1, size=(4, 13)))
    v = torch.tensor(rng.normal(0, 1, size=(4, 13)))
    term = torch.zeros(4, 13, dtype=torch.bool)
    term[:, -1] = True
    adv, tgt = o.gae(r, v, gamma=0.9, gae_lambda=1.0, terminated=term)
    ret = o.returns_to_go(r, gamma=0.9, terminated=term)
    torch.testing.assert_close(adv, ret - v)
    torch.testing.assert_close(tgt, ret)


def test_padding_invariance_ppo_and_sapo():
    rng = _rng(41)
    cur = torch.tensor(rng.normal(-1, 0.2, size=(2, 5)))
    old = cur + torch.tensor(rng.normal(0, 0.1, size=(2, 5)))
    adv = torch.tensor(rng.normal(0, 1, size=(2, 5)))
    m = torch.ones(2, 5, dtype=torch.bool)
    pad = lambda t, v: torch.cat([t, torch.full((2, 3), v, dtype=t.dtype)], dim=1)
    mp = torch.cat([m, torch.zeros(2, 3, dtype=torch.bool)], dim=1)
    a = o.ppo_clip(cur, old, adv, m)["loss"]
    b = o.ppo_clip(pad(cur, 17.0), pad(old, -12.0), pad(adv, 999.0), mp)["loss"]
    torch.testing.assert_close(a, b)
    a = o.sapo(cur, old, adv, m)["loss"]
    b = o.sapo(pad(cur, 100.0), pad(old, -100.0), pad(adv, 999.0), mp)["loss"]
    torch.testing.assert_close(a, b)


def test_gspo_equals_gspo_token_for_uniform_advantages():
    rng = _rng(42)
    cur = torch.tensor(rng.normal(0, 0.2, size=(3, 6)))
    old = torch.zeros_like(cur)
    m = torch.tensor(rng.random((3, 6)) < 0.8)
    m[:, 0] = True
    A = torch.tensor(rng.normal(0, 1, size=3))
    c1 = cur.clone().requires_grad_()
    c2 = cur.clone().requires_grad_()
    s = o.gspo(c1, old, A, m, clip_low=0.1, clip_high=0.1)
    t = o.gspo_token(c2, old, A[:, None].expand(3, 6), m, clip_low=0.1, clip_high=0.1)
    torch.testing.assert_close(s["loss"], t["loss"])
    s["loss"].backward()
    t["loss"].backward()
    torch.testing.assert_close(c1.grad, c2.grad)


def test_group_uniform_float32_groups_are_zero():
    """Uniform groups of non-dyadic float32 values standardize to exactly 0
    (advantages.py:243-244), for every group size; the float64 scalar loop
    agrees (its mean of a uniform group is exact)."""

    for v in (0.1, 0.3, 0.7, 1.0):
        for G in (2, 3, 4, 8, 16, 33, 64):
            r = torch.full((3, G), v, dtype=torch.float32)
            r[1] = torch.linspace(-1, 1, G)
            z = o.group_standardize(r)
            assert torch.equal(z[0], torch.zeros(G)) and torch.equal(z[2], torch.zeros(G))
            np.testing.assert_allclose(z.double().numpy(), brute.group_standardize(r.double()),
                                       rtol=1e-6, atol=1e-6)


def test_group_shift_invariance():
    """derivations-and-code.md:1168: adding a constant leaves centered advantages unchanged."""

    rng = _rng(43)
    r = torch.tensor(rng.normal(0, 1, size=(6, 8)))
    torch.testing.assert_close(o.group_standardize(r), o.group_standardize(r + 3.25))


# ---- planted mistakes: each mutated oracle must fail its pin -----------------


def _inclusive_trust(ratios, *, clip_low, clip_high):
    return (ratios >= 1.0 - clip_low) & (ratios <= 1.0 + clip_high)


def test_planted_inclusive_trust_bound_is_caught(monkeypatch):
    case = next(c for c in CASES if c["id"] == "double_sided_strict")
    monkeypatch.setattr(o, "strict_trust", _inclusive_trust)
    with pytest.raises(AssertionError):
        run_case(case, "oracle", "cpu")


def test_planted_optimistic_clip_is_caught():
    """max() in place of min() (the optimistic bound for negative advantages) must
    disagree with the closed-form derivative."""

    def ppo_optimistic(cur, old, adv, mask, *, clip_low=0.2, clip_high=None, max_log_ratio=20.0):
        hi = clip_low if clip_high is None else clip_high
        lr = (cur - old).clamp(-max_log_ratio, max_log_ratio)
        rho = lr.exp()
        per = torch.maximum(rho * adv, rho.clamp(1 - clip_low, 1 + hi) * adv)
        obj = o.weighted_average(per, mask)
        return {"objective": obj, "loss": -obj}

    rng = _rng(0)
    cur, old, adv, mask = _planted_inputs(rng)
    cur = old + rng.normal(0, 0.5, size=old.shape)  # plenty of ratios outside the band
    w = mask.astype(np.float64)
    _, g = _oracle_grad(ppo_optimistic, cur, old, adv, torch.tensor(w), clip_low=0.2,
                        clip_high=0.2)
    _, bg = brute.ppo_objective_grad(cur, old, adv, w, clip_low=0.2, clip_high=0.2)
    with pytest.raises(AssertionError):
        np.testing.assert_allclose(g.reshape(-1), bg, rtol=1e-12, atol=1e-15)


def test_planted_padding_as_terminal_is_caught():
    """Treating padding as a terminal (instead of absent time) breaks the padding pin."""

    r = torch.tensor([[1.0, 2.0, 999.0, 3.0]])
    valid = torch.tensor([[True, True, False, True]])
    good = o.returns_to_go(r, valid_mask=valid)
    wrong = o.returns_to_go(torch.where(valid, r, torch.zeros_like(r)), terminated=~valid)
    assert not torch.allclose(good, wrong)
    np.testing.assert_allclose(good.numpy(), brute.returns(r.numpy(), valid=valid.numpy()))


@pytest.mark.parametrize("kind", ["ppo", "sapo"])
def test_lm_head_step_vs_finite_differences(kind):
    """d hidden and d weight of the LM-head composition against central
    differences of the float64 loss in a few coordinates of each."""

    rng = _rng(11)
    B, T, H, V = 2, 5, 7, 13
    h = torch.tensor(rng.normal(0, 1.0, size=(B, T, H)))
    w = torch.tensor(rng.normal(0, 0.7, size=(V, H)))
    tgt = torch.tensor(rng.integers(0, V, size=(B, T)))
    lp0 = o.token_logprobs(h @ w.t(), tgt, exact=True)
    old = lp0 + torch.tensor(rng.normal(0, 0.1, size=(B, T)))
    adv = torch.tensor(rng.normal(0, 1, size=(B, T)))
    mask = torch.tensor(rng.random((B, T)) < 0.8)
    mask[:, 0] = True
    kw = dict(clip_low=0.2, clip_high=0.28) if kind == "ppo" else {}
    out, _lp, dh, dw = o.lm_head_step(kind, h, w, h @ w.t(), tgt, old, adv, mask, exact=True,
                                      **kw)

    def loss(hh, ww):
        o2, _, _ = o.policy_step(kind, hh @ ww.t(), tgt, old, adv, mask, exact=True, **kw)
        return float(o2["loss"])

    assert abs(loss(h, w) - float(out["loss"])) < 1e-14
    eps = 1e-6
    for idx in [(0, 0, 0), (1, 3, 6), (0, 4, 2)]:
        e = torch.zeros_like(h)
        e[idx] = eps
        fd = (loss(h + e, w) - loss(h - e, w)) / (2 * eps)
        assert abs(fd - float(dh[idx])) <= 1e-7 * max(1.0, abs(fd)), (idx, fd, float(dh[idx]))
    for idx in [(0, 0), (int(tgt[0, 1]), 3), (12, 6)]:
        e = torch.zeros_like(w)
        e[idx] = eps
        fd = (loss(h, w + e) - loss(h, w - e)) / (2 * eps)
        assert abs(fd - float(dw[idx])) <= 1e-7 * max(1.0, abs(fd)), (idx, fd, float(dw[idx]))
