"""The sampling oracle (roseinfer/engine.py:1103-1171) pinned on the CPU.

* Philox4x32-10 against the known-answer vectors published with the Random123
  library (the generator the kernel draws its uniforms from), for the oracle
  and for the library's own host copy of the generator;
* the sampling distribution against a direct restatement of the reference's
  torch op chain (topk / softmax / cumsum / masked_fill / clamp_min) in
  float64 on tie-free logits;
* the inverse-CDF draw against the distribution by a chi-square test, and the
  uniforms by their first two moments and a Kolmogorov-Smirnov bound.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest
import torch

from oracle import sampler_oracle as so

KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_philox_known_answers(ctr, key, want):
    assert so.philox4x32_10(ctr, key) == want


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_library_philox_known_answers(ctr, key, want):
    from rosellm_amd import _native as nat

    lib = nat.load()
    c = (ctypes.c_uint32 * 4)(*ctr)
    k = (ctypes.c_uint32 * 2)(*key)
    lib.rrl_philox4x32_10(c, k)
    assert tuple(c) == want


def _reference_chain(x: torch.Tensor, T: float, top_k: int, top_p: float) -> torch.Tensor:
    """engine.py:1141-1171's PyTorch path, restated on float64: the unnormalised
    probabilities torch.multinomial receives, scattered back to vocabulary ids."""

    V = x.numel()
    scaled = (x / T)[None]
    q = torch.zeros(V, dtype=torch.float64)
    if top_p <= 0.0 or top_p >= 1.0:
        if top_k <= 0 or top_k >= V:
            return torch.softmax(scaled, dim=-1).clamp_min(1e-9)[0]
        vals, idx = torch.topk(scaled, min(top_k, V), dim=-1)
        q[idx[0]] = torch.softmax(vals, dim=-1).clamp_min(1e-9)[0]
        return q
    k = V if top_k <= 0 else min(top_k, V)
    sorted_logits, sorted_idx = torch.topk(scaled, k, dim=-1)
    probs = torch.softmax(sorted_logits, dim=-1)
    cum = torch.cumsum(probs, dim=-1)
    mask = cum > float(top_p)
    mask[..., 0] = False
    probs = probs.masked_fill(mask, 0.0).clamp_min(1e-9)
    q[sorted_idx[0]] = probs[0]
    return q


CASES = [(1.0, 0, 1.0), (0.7, 50, 1.0), (1.3, 0, 0.9), (1.0, 20, 0.5), (1.0, 0, 0.05),
         (2.0, 4000, 0.95), (0.5, 1, 1.0), (1.0, 5000, 1.0)]


@pytest.mark.parametrize("T,top_k,top_p", CASES)
def test_distribution_matches_reference_chain(T, top_k, top_p):
    g = torch.Generator().manual_seed(17)
    for _ in range(3):
        x = torch.randn(5000, generator=g, dtype=torch.float64) * 2.5
        want = _reference_chain(x, T, top_k, top_p)
        got, cand = so.sampling_distribution(x.numpy(), T, top_k, top_p)
        np.testing.assert_allclose(got, want.numpy(), rtol=1e-12, atol=1e-20)
        assert cand.sum() == (top_k if 0 < top_k < 5000 else 5000)


def test_inverse_cdf_draws_follow_the_distribution():
    V, B = 24, 40000
    x = np.random.default_rng(3).normal(size=V) * 1.5
    q, _ = so.sampling_distribution(x, 1.0, 0, 1.0)
    rows = np.broadcast_to(x, (B, V))
    out = so.sample_rows(rows, temperature=1.0, top_k=0, top_p=1.0, do_sample=True,
                         seed=99, offset=5)
    counts = np.bincount(out["token"], minlength=V)
    expect = q / q.sum() * B
    chi2 = float((((counts - expect) ** 2) / expect).sum())
    # chi-square with 23 degrees of freedom: P(chi2 > 60) ~ 3e-5
    assert chi2 < 60.0, chi2
    np.testing.assert_allclose(out["logq"], np.log(q[out["token"]] / q.sum()), rtol=1e-12)


@pytest.mark.parametrize("p", [
    [5e-10, 2e-10, 3e-9, 1e-10, 0.0, 4e-9],
    [1e-9, 7e-10, 7e-10, 2e-9],
    [3e-10, 3e-10, 3e-10],  # every entry floored: p itself has the smaller share
])
def test_mixture_rule_draws_the_floored_weights(p):
    """The plain-sampling draw of max(p, 1e-9) as a mixture of p and the
    floor's excess, integrated exactly over both uniforms.  Weights this small
    give the floor a large share, so a wrong component probability, swapped
    components or a wrong excess changes the frequencies by far more than the
    grid's resolution.  The frequencies must be max(p, 1e-9) / sum."""

    p = np.asarray(p, dtype=np.float64)
    q = np.maximum(p, 1e-9)
    want = q / q.sum()
    n = 4000
    grid = (np.arange(n) + 0.5) / n
    freq = np.zeros(p.size)
    rho, g, pi = so.mixture_parts(p)
    assert math.isclose(pi, g.sum() / (p.sum() + g.sum()), rel_tol=1e-15)
    # u1 picks the component; u the position inside it: the frequencies of a
    # grid over (u1, u) are pi * (grid draws of g) + (1 - pi) * (grid of p)
    for comp, share in ((g, pi), (rho, 1.0 - pi)):
        if share == 0.0:
            continue
        toks = np.array([so.inverse_cdf(comp, u)[0] for u in grid])
        freq += share * np.bincount(toks, minlength=p.size) / n
    np.testing.assert_allclose(freq, want, atol=2.0 / n)
    # and mixture_draw picks the component the same way
    for u1 in (0.0, pi * 0.999, pi * 1.001, 0.999999):
        tok, _ = so.mixture_draw(p, 0.5, u1)
        assert tok == so.inverse_cdf(g if u1 < pi else rho, 0.5)[0]


def _grid_freq(p, rule, n=4000):
    """Frequencies of a two-component rule (weights a, b, probability of a)
    integrated over a grid of both uniforms."""

    p = np.asarray(p, dtype=np.float64)
    grid = (np.arange(n) + 0.5) / n
    a, b, pa = rule(p)
    freq = np.zeros(p.size)
    for comp, share in ((a, pa), (b, 1.0 - pa)):
        if share > 0.0:
            toks = np.array([so.inverse_cdf(comp, u)[0] for u in grid])
            freq += share * np.bincount(toks, minlength=p.size) / n
    return freq


@pytest.mark.parametrize("mistake", ["swapped components", "pi of p", "no floor excess"])
def test_mixture_check_catches_planted_mistakes(mistake):
    """The frequency check of the mixture rule fails for plausible mistakes
    planted in the rule (on the CPU): the excess drawn with p's probability,
    the components' probabilities taken as S / (S + G), or the excess
    dropped."""

    p = np.array([5e-10, 2e-10, 3e-9, 1e-10, 0.0, 4e-9])
    want = np.maximum(p, 1e-9) / np.maximum(p, 1e-9).sum()

    def right(p):
        rho, g, pi = so.mixture_parts(p)
        return g, rho, pi

    def wrong(p):
        rho, g, pi = so.mixture_parts(p)
        if mistake == "swapped components":
            return rho, g, pi
        if mistake == "pi of p":
            return g, rho, 1.0 - pi
        return g, rho, 0.0

    tol = 2.0 / 4000
    assert np.allclose(_grid_freq(p, right), want, atol=tol)
    assert not np.allclose(_grid_freq(p, wrong), want, atol=tol)


def test_inverse_cdf_edges():
    # the target lands on a boundary: the next entry with positive weight
    w = np.array([0.25, 0.0, 0.25, 0.5])
    assert so.inverse_cdf(w, 0.25)[0] == 2
    assert so.inverse_cdf(w, 0.0)[0] == 0
    assert so.inverse_cdf(w, 0.9999)[0] == 3
    # rounding past the end takes the last positive entry, not a zero one
    assert so.inverse_cdf(np.array([0.5, 0.5, 0.0]), 1.0)[0] == 1


def test_uniforms():
    u1 = np.array([so.row_uniforms(1234, 7, r)[1] for r in range(50000)])
    assert abs(u1.mean() - 0.5) < 0.005 and abs(u1.var() - 1 / 12) < 0.002
    # the component uniform takes bits the position uniform does not use
    w = so.philox4x32_10((3, 0, 7, 0), (1234, 0))
    assert so.row_uniforms(1234, 7, 3)[1] * 2.0 ** 53 == (w[1] << 21) | (w[2] >> 11)
    u = np.array([so.row_uniform(1234, 7, r) for r in range(50000)])
    assert abs(u.mean() - 0.5) < 0.005 and abs(u.var() - 1 / 12) < 0.002
    ks = np.max(np.abs(np.sort(u) - (np.arange(u.size) + 0.5) / u.size))
    assert ks < 1.63 / math.sqrt(u.size)  # 1% critical value
    # different offsets / seeds give different streams
    assert so.row_uniform(1234, 8, 0) != so.row_uniform(1234, 7, 0)
    assert so.row_uniform(1235, 7, 0) != so.row_uniform(1234, 7, 0)


def test_greedy_and_first_token_rules():
    x = np.array([[0.5, 2.0, 2.0, -1.0]])
    out = so.sample_rows(x, temperature=0.0, top_k=0, top_p=1.0, do_sample=True, seed=1, offset=0)
    assert out["token"][0] == 1 and out["logq"][0] == 0.0
    # top_p below the largest probability keeps only the first token (plus
    # the 1e-9 floor on the others)
    q, _ = so.sampling_distribution(np.array([3.0, 0.0, -1.0]), 1.0, 0, 1e-6)
    assert q[1] == q[2] == 1e-9 and q[0] > 0.9
    # top-k ties: lowest index first
    _, cand = so.sampling_distribution(np.array([1.0, 5.0, 1.0, 1.0, 0.0]), 1.0, 3, 1.0)
    assert cand.tolist() == [True, True, True, False, False]


def test_top_p_margin():
    """Distance of top_p from the cumulative masses either side of the cut,
    on hand-computed distributions."""
    x = np.log(np.array([0.5, 0.3, 0.2]))
    assert so.top_p_margin(x, 1.0, 0, 1.0) == math.inf
    # cum 0.5 | 0.8 | 1.0: at 0.7 the cut lies between 0.5 (kept) and 0.8
    assert math.isclose(so.top_p_margin(x, 1.0, 0, 0.7), 0.1, rel_tol=1e-9)
    # top_p on a cumulative mass: the cut is undecided
    assert so.top_p_margin(x, 1.0, 0, 0.8) < 1e-12
    # top-k 2 renormalises 0.4, 0.3 to 4/7, 3/7: at 0.6 the nearest is 4/7
    x = np.log(np.array([0.1, 0.4, 0.2, 0.3]))
    assert math.isclose(so.top_p_margin(x, 1.0, 2, 0.6), 0.6 - 4 / 7, rel_tol=1e-9)
    # temperature 2 flattens 0.5/0.3/0.2 before the cut
    x = np.log(np.array([0.5, 0.3, 0.2]))
    p = np.sqrt([0.5, 0.3, 0.2]); p /= p.sum()
    assert math.isclose(so.top_p_margin(x, 2.0, 0, 0.5), min(p[0] + p[1] - 0.5, 0.5 - p[0]),
                        rel_tol=1e-9)

