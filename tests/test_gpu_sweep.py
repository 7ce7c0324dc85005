"""Seeded random sweep of the single-pass path and the SFT loss against the
float64 oracle (MI355X): every dtype, tiny and odd vocabularies (V = 1, 7, 9;
the register-resident kernel from V = 8 up), causal-shift and batch-strided
views, int32 / int64 targets, float and bool masks, every objective.  Bars as
in test_gpu_parity (log-probs 1e-5; losses 1e-5 / 2e-3 for 16-bit against the
terms' scale; dlogits 1e-5 of |g| per row for float32/64, row-norm 2e-3 and
one ulp for 16-bit)."""

from __future__ import annotations

import random

import pytest
import torch

from oracle import roserlhf_oracle as o
from rosellm_amd import roserlhf as R
from rosellm_amd import rosetrainer as RT

from test_gpu_parity import F32_RTOL, _close, _close_rows_by_g, _rownorm16, _ulp16

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16, torch.float32, torch.float64]
VOCABS = [1, 2, 7, 8, 9, 64, 1000, 4096, 8200, 30001, 65536, 151936]
OBJECTIVES = ["clipped", "sao", "sapo", "gspo", "gspo_token", "nll"]
KW = {"clipped": dict(clip_low=0.2, clip_high=0.28), "sao": dict(clip_low=0.2, clip_high=0.28),
      "sapo": dict(tau_positive=1.0, tau_negative=1.05),
      "gspo": dict(clip_low=3e-4, clip_high=4e-4), "gspo_token": dict(clip_low=3e-4, clip_high=4e-4)}


def _case(i):
    rng = random.Random(7000 + i)
    dtype = DTYPES[i % 4]
    V = rng.choice(VOCABS if dtype != torch.float64 else VOCABS[:9])
    objective = OBJECTIVES[(i // 4) % len(OBJECTIVES)]
    B = rng.randint(1, 5)
    T = rng.choice([1, 2, 5, 17, 40])
    layout = rng.choice(["contiguous", "shift", "batch_slice"])
    tdtype = rng.choice([torch.int64, torch.int32])
    mask_kind = rng.choice(["bool", "float"])
    return dict(seed=7000 + i, dtype=dtype, V=V, objective=objective, B=B, T=T, layout=layout,
                tdtype=tdtype, mask_kind=mask_kind)


CASES = [_case(i) for i in range(192)]


def _ids(c):
    return (f"{c['objective']}-{str(c['dtype'])[6:]}-V{c['V']}-B{c['B']}T{c['T']}-{c['layout']}"
            f"-{str(c['tdtype'])[6:]}-{c['mask_kind']}")


@pytest.mark.parametrize("c", CASES, ids=_ids)
def test_sweep(device, c):
    print(f"[sweep] {_ids(c)}", flush=True)
    g = torch.Generator().manual_seed(c["seed"])
    B, T, V, dtype = c["B"], c["T"], c["V"], c["dtype"]
    # the logits tensor the caller holds, and the [B, T, V] rows the loss reads
    if c["layout"] == "shift":
        full = torch.randn(B, T + 1, V, generator=g) * 3.0
        rows = lambda z: z[:, :-1]
    elif c["layout"] == "batch_slice":
        full = torch.randn(2 * B, T, V, generator=g) * 3.0
        rows = lambda z: z[::2]
    else:
        full = torch.randn(B, T, V, generator=g) * 3.0
        rows = lambda z: z
    hot = torch.rand(full.shape[:-1], generator=g) < 0.1
    col = torch.randint(0, V, full.shape[:-1], generator=g)
    full[hot, col[hot]] += 15.0
    full = full.to(dtype)
    x = rows(full)
    t = torch.randint(0, V, (B, T), generator=g)
    lengths = torch.randint(1, T + 1, (B,), generator=g)
    mask = torch.arange(T)[None, :] < lengths[:, None]
    if c["mask_kind"] == "float":
        mask = mask.to(torch.float32)
    lp0 = o.token_logprobs(x, t)
    old = (lp0 + torch.randn(B, T, generator=g) * 0.1).float()
    adv = torch.randn(B, T, generator=g)
    objective = c["objective"]
    fd = full.to(device).requires_grad_()
    d = lambda z: z.to(device)

    if objective == "nll":
        labels = t.clone()
        labels[torch.rand(B, T, generator=g) < 0.2] = -100
        labels[0, 0] = t[0, 0]  # at least one scored token (else the mean is NaN)
        loss = RT.cross_entropy(rows(fd), d(labels).to(c["tdtype"]))
        loss.backward()
        want, dlo = o.sft_step(x, labels, causal=False, exact=True)
        n = int((labels != -100).sum())
        gabs = torch.where(labels != -100, torch.full((B, T), 1.0 / max(n, 1)), torch.zeros(B, T))
        got_loss, want_loss, scale = loss.item(), want.item(), abs(want.item())
    else:
        a = adv[:, 0].contiguous() if objective == "gspo" else adv
        out, lp = R.fused_policy_loss(rows(fd), d(t).to(c["tdtype"]), d(old), d(a), d(mask),
                                      objective=objective, return_logprobs=True, **KW[objective])
        out.loss.backward()
        kind = {"clipped": "ppo"}.get(objective, objective)
        out_o, lpo, dlo = o.policy_step(kind, x, t, old, a, mask, exact=True, **KW[objective])
        _close(lp, lpo, F32_RTOL, 1e-7, "logp")
        gabs = out_o["dloss_dlogp"]
        got_loss, want_loss = out.loss.item(), out_o["loss"].item()
        scale = max(abs(want_loss), a.abs().mean().item())
    rt = F32_RTOL if dtype in (torch.float32, torch.float64) else 2e-3
    assert abs(got_loss - want_loss) <= rt * scale + 1e-12, (got_loss, want_loss)
    grad = rows(fd.grad)
    if c["layout"] == "shift":
        assert (fd.grad[:, -1] == 0).all()
    if c["layout"] == "batch_slice":
        assert (fd.grad[1::2] == 0).all()
    if dtype in (torch.float32, torch.float64):
        _close_rows_by_g(grad, dlo, gabs, F32_RTOL, "dlogits")
    else:
        assert _ulp16(grad, dlo, "dlogits") > 0.98 or V <= 9
        _rownorm16(grad, dlo, 2e-3, "dlogits")
