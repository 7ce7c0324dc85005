"""Seeded random sweep of the fused LM-head path (config 5's entry point)
against the CPU oracle (MI355X): every objective, bf16 and float32, hidden
sizes 16-128, vocabularies from 7 to 8256 entries, row blocks from one token
(a sequence cut into one-token stretches) to whole batches, with and without
skip_masked_rows.  Bars as in test_gpu_linear: log-probs within 1e-5 of the
float64 oracle on the same rounded block products; the loss within 2e-3
(bf16) or 1e-5 (float32) of the terms' scale; bf16 d hidden / d weight within
the bound one-ulp dlogits deviations can move them, float32 rows within 1e-5."""

from __future__ import annotations

import random

import pytest
import torch

from oracle import roserlhf_oracle as o
from rosellm_amd import roserlhf as R

from test_gpu_linear import KW, _inputs, _product_check, _rows_close

pytestmark = pytest.mark.gpu

OBJECTIVES = ["clipped", "sao", "sapo", "gspo", "gspo_token"]


def _case(i):
    rng = random.Random(8800 + i)
    return dict(seed=8800 + i, dtype=[torch.bfloat16, torch.float32][i % 2],
                objective=OBJECTIVES[(i // 2) % len(OBJECTIVES)], B=rng.choice([4, 8]),
                T=rng.choice([1, 3, 17, 100]), H=rng.choice([16, 64, 128]),
                V=rng.choice([7, 64, 1000, 4099, 8256]), row_block=rng.choice([1, 5, 64, 192, 4096]),
                skip=rng.choice([False, True]))


CASES = [_case(i) for i in range(40)]


def _ids(c):
    return (f"{c['objective']}-{str(c['dtype'])[6:]}-B{c['B']}T{c['T']}H{c['H']}V{c['V']}-"
            f"rb{c['row_block']}-{'skip' if c['skip'] else 'all'}")


@pytest.mark.parametrize("c", CASES, ids=_ids)
def test_linear_sweep(device, c):
    print(f"[linear sweep] {_ids(c)}", flush=True)
    B, T, H, V, rb = c["B"], c["T"], c["H"], c["V"], c["row_block"]
    h, w, x, t, old, adv, mask = _inputs(c["seed"], B, T, H, V, c["dtype"], device, rb)
    objective = c["objective"]
    kw = KW[objective]
    a = adv[:, 0].contiguous() if objective == "gspo" else adv
    hd = h.to(device).requires_grad_()
    wd = w.to(device).requires_grad_()
    d = lambda z: z.to(device)  # noqa: E731
    # skip_masked_rows: token-local objectives only, and without log-probs
    # (masked rows are never read)
    skip = c["skip"] and objective in ("clipped", "sao", "sapo")
    res = R.fused_linear_policy_loss(hd, wd, d(t), d(old), d(a), d(mask), objective=objective,
                                     return_logprobs=not skip, row_block=rb,
                                     skip_masked_rows=skip, **kw)
    out, lp = (res, None) if skip else res
    out.loss.backward()
    kind = {"clipped": "ppo"}.get(objective, objective)
    out_o, lpo, dho, dwo = o.lm_head_step(kind, h, w, x, t, old, a, mask, exact=True, **kw)
    if lp is not None:
        err = (lp.detach().cpu().double() - lpo).abs()
        assert bool((err <= 1e-5 * lpo.abs() + 1e-7).all()), float(err.max())
    scale = max(abs(out_o["loss"].item()), a.abs().mean().item())
    rt = 2e-3 if c["dtype"] == torch.bfloat16 else 1e-5
    assert abs(out.loss.item() - out_o["loss"].item()) <= rt * scale, (
        out.loss.item(), out_o["loss"].item())
    if c["dtype"] == torch.bfloat16:
        dl16 = out_o["dlogits"].double().reshape(-1, V)
        _product_check(hd.grad.reshape(-1, H), dl16, w, "dhidden", transpose=False)
        _product_check(wd.grad, dl16, h.reshape(-1, H), "dweight", transpose=True)
    else:
        _rows_close(hd.grad.reshape(-1, H), dho.reshape(-1, H), 1e-5, "dhidden f32")
        _rows_close(wd.grad, dwo, 1e-5, "dweight f32")
