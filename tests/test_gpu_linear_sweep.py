"""Seeded random sweep of the matrix-core LM head (config 5's entry point)
against the CPU oracle (MI355X), through both implementations: every
objective, hidden sizes 128-1024 (both tile-load layouts of the tile path),
vocabularies from 1 to 8256 entries, token counts that are not 64-row block
multiples, one-token sequences, row blocks of the chunked path that cut the
batch into several.  Bars as in test_gpu_linear: log-probs against the float64
oracle on the logits each implementation consumed (the chunked path's
recorded and pinned to the exact products); the loss within 2e-3 of
the terms' scale; d hidden / d weight within twice the bound one-ulp bf16
dlogits deviations can move them."""

from __future__ import annotations

import random

import pytest
import torch

from rosellm_amd import roserlhf as R

from test_gpu_linear import (IMPLS, KW, _inputs, _logp_check_impl, _oracle_step, _product_check,
                             _tap)

pytestmark = pytest.mark.gpu

OBJECTIVES = ["clipped", "sao", "sapo", "gspo", "gspo_token"]


def _case(i):
    rng = random.Random(8800 + i)
    return dict(seed=8800 + i, objective=OBJECTIVES[i % len(OBJECTIVES)],
                B=rng.choice([4, 8]), T=rng.choice([1, 3, 17, 100]),
                H=rng.choice([128, 256, 384, 640, 1024]),
                V=rng.choice([1, 7, 64, 1000, 4099, 8256]),
                row_block=rng.choice([16384, 64, 29]))


CASES = [_case(i) for i in range(30)]


def _ids(c):
    return f"{c['objective']}-B{c['B']}T{c['T']}H{c['H']}V{c['V']}rb{c['row_block']}"


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("c", CASES, ids=_ids)
def test_linear_sweep(device, c, impl):
    print(f"[linear sweep] {impl} {_ids(c)}", flush=True)
    B, T, H, V = c["B"], c["T"], c["H"], c["V"]
    h, w, x, t, old, adv, mask = _inputs(c["seed"], B, T, H, V)
    objective = c["objective"]
    kw = KW[objective]
    a = adv[:, 0].contiguous() if objective == "gspo" else adv
    hd = h.to(device).requires_grad_()
    wd = w.to(device).requires_grad_()
    d = lambda z: z.to(device)  # noqa: E731
    with _tap(impl) as rec:
        out, lp = R.fused_linear_policy_loss(hd, wd, d(t), d(old), d(a), d(mask),
                                             objective=objective, return_logprobs=True,
                                             impl=impl, row_block=c["row_block"], **kw)
        out.loss.backward()
    kind = {"clipped": "ppo"}.get(objective, objective)
    _logp_check_impl(impl, lp, x, t, rec, h, w)
    out_o = _oracle_step(impl, kind, h, w, x, t, old, a, mask, rec, **kw)
    scale = max(abs(out_o["loss"].item()), a.abs().mean().item())
    assert abs(out.loss.item() - out_o["loss"].item()) <= 2e-3 * scale, (
        out.loss.item(), out_o["loss"].item())
    dl = out_o["dlogits"].double().reshape(-1, V)  # float64 on the consumed logits
    _product_check(hd.grad.reshape(-1, H), dl, w, "dhidden", transpose=False)
    _product_check(wd.grad, dl, h.reshape(-1, H), "dweight", transpose=True)
