"""Seeded random sweep of the return and advantage estimators against the
oracle (MI355X): returns-to-go, GAE and skip-observation GAE over random
lengths (1 to 4097 steps), batch ranks 1-3, contiguous, transposed and
sliced views, gamma / lambda at and between 0 and 1, padding and terminal
densities from none to all, with and without a bootstrap; group
standardization and leave-one-out over random group sizes on either
dimension; turn broadcast and masked whitening.  float32 results within 1e-5
of the largest magnitude (the device scans reassociate the recurrence),
float64 within 1e-12; broadcast bit-exact."""

from __future__ import annotations

import random

import pytest
import torch

from oracle import roserlhf_oracle as o
from rosellm_amd import roserlhf as R

from test_gpu_parity import F32_RTOL, _close

pytestmark = pytest.mark.gpu


def _case(i):
    rng = random.Random(4400 + i)
    return dict(
        seed=4400 + i, dtype=[torch.float32, torch.float64][i % 2],
        T=rng.choice([1, 2, 3, 31, 64, 255, 1000, 4097]),
        batch=rng.choice([(), (1,), (4,), (2, 3)]),
        layout=rng.choice(["contiguous", "transposed", "sliced"]),
        gamma=rng.choice([1.0, 0.99, 0.5, 0.0]), lam=rng.choice([1.0, 0.95, 0.0]),
        valid=rng.choice([1.0, 0.8, 0.3, 0.0]), term=rng.choice([0.0, 0.02, 0.3]),
        boot=rng.choice([False, True]))


CASES = [_case(i) for i in range(96)]


def _ids(c):
    return (f"{str(c['dtype'])[6:]}-T{c['T']}-b{'x'.join(map(str, c['batch'])) or '0'}-"
            f"{c['layout']}-g{c['gamma']}-l{c['lam']}-v{c['valid']}-d{c['term']}-"
            f"{'boot' if c['boot'] else 'noboot'}")


def _view(x, layout, device):
    """x on the device, as a contiguous, transposed or sliced view."""

    if layout == "contiguous" or x.ndim < 2:
        return x.to(device)
    if layout == "transposed":
        return x.transpose(-1, -2).contiguous().to(device).transpose(-1, -2)
    wide = torch.zeros(*x.shape[:-1], 2 * x.shape[-1], dtype=x.dtype)
    wide[..., ::2] = x
    return wide.to(device)[..., ::2]


def _tol(want, dtype):
    rtol = 1e-12 if dtype == torch.float64 else F32_RTOL
    return rtol, rtol * max(1.0, want.abs().max().item() if want.numel() else 1.0)


@pytest.mark.parametrize("c", CASES, ids=_ids)
def test_returns_and_gae_sweep(device, c):
    print(f"[estimator sweep] {_ids(c)}", flush=True)
    g = torch.Generator().manual_seed(c["seed"])
    shape = (*c["batch"], c["T"])
    dt = c["dtype"]
    r = torch.randn(shape, generator=g, dtype=torch.float64).to(dt)
    v = torch.randn(shape, generator=g, dtype=torch.float64).to(dt)
    valid = torch.rand(shape, generator=g) < c["valid"]
    term = torch.rand(shape, generator=g) < c["term"]
    boot = (torch.randn(c["batch"], generator=g, dtype=torch.float64).to(dt)
            if c["boot"] else None)
    d = lambda t: None if t is None else _view(t, c["layout"], device)  # noqa: E731
    kw = dict(terminated=term, valid_mask=valid)
    dkw = dict(terminated=d(term), valid_mask=d(valid))
    bd = None if boot is None else boot.to(device)

    got = R.discounted_returns(d(r), gamma=c["gamma"], bootstrap_value=bd, **dkw)
    want = o.returns_to_go(r, gamma=c["gamma"], bootstrap_value=boot, **kw)
    _close(got, want, *_tol(want, dt), "returns")

    ga, gt = R.generalized_advantage_estimation(d(r), d(v), gamma=c["gamma"], gae_lambda=c["lam"],
                                                bootstrap_value=bd, **dkw)
    wa, wt = o.gae(r, v, gamma=c["gamma"], gae_lambda=c["lam"], bootstrap_value=boot, **kw)
    _close(ga, wa, *_tol(wa, dt), "gae advantages")
    _close(gt, wt, *_tol(wt, dt), "gae targets")

    n = torch.roll(v, -1, dims=-1)
    sa, st = R.skip_observation_generalized_advantage_estimation(
        d(r), d(v), d(n), gamma=c["gamma"], gae_lambda=c["lam"], **dkw)
    wa, wt = o.skip_observation_gae(r, v, n, gamma=c["gamma"], gae_lambda=c["lam"], **kw)
    _close(sa, wa, *_tol(wa, dt), "skip-observation advantages")
    _close(st, wt, *_tol(wt, dt), "skip-observation targets")



@pytest.mark.parametrize("i", range(24))
def test_group_estimators_sweep(device, i):
    rng = random.Random(5500 + i)
    dt = [torch.float32, torch.float64][i % 2]
    G, n = rng.choice([1, 3, 64, 1000]), rng.choice([1, 2, 5, 16, 64])
    dim = rng.choice([-1, 0])
    print(f"[group sweep] {dt} G={G} n={n} dim={dim}", flush=True)
    g = torch.Generator().manual_seed(5500 + i)
    r = torch.randn(G, n, generator=g, dtype=torch.float64).to(dt)
    r[0] = 1.0  # a uniform group
    if G > 2:
        r[1] = torch.randint(0, 2, (n,), generator=g).to(dt)  # binary rewards
        # uniform groups of non-dyadic values: exactly zero, whose float mean
        # is often an ulp off the value itself
        r[2] = [0.1, 0.3, 0.7][i % 3]
    x = r if dim == -1 else r.t().contiguous()
    if n < 2:  # the reference's rule (advantages.py:230-231, 250-251)
        with pytest.raises(ValueError, match="group standardization requires group_size >= 2"):
            R.group_standardized_advantages(x.to(device), dim=dim)
        with pytest.raises(ValueError, match="leave-one-out advantages require group_size >= 2"):
            R.leave_one_out_advantages(x.to(device), dim=dim)
        return
    got = R.group_standardized_advantages(x.to(device), dim=dim)
    want = o.group_standardize(x, dim=dim)
    _close(got, want, *_tol(want, dt), "group standardize")
    uni = [0, 2] if G > 2 else [0]
    got_rows = got.cpu() if dim == -1 else got.cpu().t()
    assert (got_rows[uni] == 0).all(), "a uniform group must standardize to exactly zero"
    got = R.leave_one_out_advantages(x.to(device), dim=dim)
    want = o.leave_one_out(x, dim=dim)
    _close(got, want, *_tol(want, dt), "leave one out")


@pytest.mark.parametrize("i", range(16))
def test_turn_broadcast_and_whiten_sweep(device, i):
    rng = random.Random(6600 + i)
    B, T, K = rng.choice([1, 3, 17]), rng.choice([1, 7, 300, 5000]), rng.choice([1, 2, 9])
    dens = rng.choice([0.0, 0.3, 1.0])
    print(f"[turn/whiten sweep] B={B} T={T} K={K} mask={dens}", flush=True)
    g = torch.Generator().manual_seed(6600 + i)
    ta = torch.randn(B, K, generator=g)
    ids = torch.randint(0, K, (B, T), generator=g)
    m = torch.rand(B, T, generator=g) < dens
    ids[~m] = -1 - torch.randint(0, 3, (B, T), generator=g)[~m]  # any id where masked
    got = R.broadcast_turn_advantages(ta.to(device), ids.to(device), m.to(device)).cpu()
    assert torch.equal(got, o.turn_broadcast(ta, ids, m))
    if bool(m.any()):
        x = torch.randn(B, T, generator=g) * 3 + 1
        for shift in (True, False):
            got = R.masked_whiten(x.to(device), m.to(device), shift_mean=shift)
            want = o.masked_whiten(x, m, shift_mean=shift)
            _close(got, want, 1e-5, 1e-5 * max(1.0, want.abs().max().item()), "whiten")
