"""Fused LM-head path (config 5) vs the CPU oracle on identical seeded inputs.

The logits product is the GEMM library's (hipBLASLt through torch.mm): the
oracle is fed the same rounded row-block products the path consumed, computed
here with torch.mm over the same row blocks, and runs the rest of the chain in
float64 (``lm_head_step``).  Bars, as for the logits-level path:

* log-probs within 1e-5 relative of the float64 oracle;
* the loss within 2e-3 of the objective's term scale (bf16 inputs);
* d hidden and d weight (bf16): the reference's autograd feeds the linear
  map's backward bf16 dlogits, and the row kernels hold each dlogit within
  one ulp of the correctly rounded exact value (the logits-level bar).  So
  every element of ``dlogits16 @ W`` / ``dlogits16.T @ hidden`` must lie
  within what those one-ulp deviations can move it (``ulp(dlogits16) @ |W|``,
  resp. ``ulp(dlogits16).T @ |hidden|``) plus one ulp of the bf16 output,
  around the float64 product of the correctly rounded dlogits; and 99% of
  the rows within 2e-3 norm-wise of that product rounded to bf16.  A row of
  dW fed by a handful of dominant tokens moves by up to 2^-8 when one of
  their dlogits sits one ulp away, so the bar is the propagated bound, not a
  flat row-norm tolerance;
* float32 inputs: every row of d hidden and d weight within 1e-5 norm-wise.
"""

from __future__ import annotations

import pytest
import torch

from oracle import roserlhf_oracle as o
from rosellm_amd import roserlhf as R
from rosellm_amd.roserlhf import linear as LIN

pytestmark = pytest.mark.gpu

KW = {"clipped": dict(clip_low=0.2, clip_high=0.28), "sao": dict(clip_low=0.2, clip_high=0.28),
      "sapo": dict(tau_positive=1.0, tau_negative=1.05),
      "gspo": dict(clip_low=3e-4, clip_high=4e-4), "gspo_token": dict(clip_low=3e-4, clip_high=4e-4)}


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _partition(B, T, row_block):
    """The row blocks the path uses, restated: whole sequences per block when
    a sequence fits, else stretches of one sequence."""

    if T <= row_block:
        bc = max(1, row_block // T)
        return [(b0, min(B, b0 + bc), 0, T) for b0 in range(0, B, bc)]
    return [(b, b + 1, t0, min(T, t0 + row_block)) for b in range(B) for t0 in range(0, T, row_block)]


def _block_logits(h, w, row_block):
    """[B, T, V] products, one torch.mm per row block (as the path forms them)."""

    B, T, H = h.shape
    h2 = h.reshape(B * T, H)
    parts = []
    for b0, b1, t0, t1 in _partition(B, T, row_block):
        r0, n = b0 * T + t0, (b1 - b0) * (t1 - t0)
        parts.append(torch.mm(h2[r0:r0 + n], w.t()))
    return torch.cat(parts).reshape(B, T, -1)


def _inputs(seed, B, T, H, V, dtype, device, row_block):
    g = _gen(seed)
    h = torch.randn(B, T, H, generator=g).to(dtype)
    w = (torch.randn(V, H, generator=g) * (2.0 / H ** 0.5)).to(dtype)
    hd, wd = h.to(device), w.to(device)
    x = _block_logits(hd, wd, row_block).cpu()
    probs = torch.softmax(x.double(), dim=-1)
    t = torch.multinomial(probs.reshape(-1, V), 1, generator=g).reshape(B, T)
    lp = o.token_logprobs(x, t, exact=True).float()
    old = lp + torch.randn(B, T, generator=g) * 0.1
    lengths = torch.randint(1, T + 1, (B,), generator=g)
    mask = torch.arange(T)[None, :] < lengths[:, None]
    r = torch.randint(0, 2, (B // 4, 4), generator=g).float()
    adv = o.group_standardize(r).reshape(-1)[:, None].expand(B, T).contiguous()
    return h, w, x, t, old, adv, mask


def _rows_close(got, want, tol, what):
    """Row-norm relative error against float64 rows (float32 outputs)."""

    g = got.detach().cpu().double().reshape(-1, got.shape[-1])
    w = want.detach().cpu().double().reshape(-1, got.shape[-1])
    den = w.norm(dim=-1)
    rel = torch.where(den > 0, (g - w).norm(dim=-1) / den.clamp_min(1e-300), (g - w).norm(dim=-1))
    worst = float(rel.max())
    print(f"{what}: worst row-norm rel err {worst:.3e}", flush=True)
    assert worst <= tol, f"{what}: worst row-norm rel err {worst:.3e} > {tol}"


def _ulp16(v):
    """bf16 unit in the last place of each (bf16-representable) value."""

    m, e = torch.frexp(v.double())
    return torch.where(v != 0, torch.ldexp(torch.ones_like(m), e - 8), torch.zeros_like(m))


def _product_check(got, dl16, other, what, transpose):
    """got = bf16 GEMM of the kernel's dlogits with ``other``; dl16: the
    correctly rounded exact dlogits [rows, V] (float64 copy)."""

    a = dl16.t() if transpose else dl16
    ref = a @ other.double()
    prop = (_ulp16(dl16).t() if transpose else _ulp16(dl16)) @ other.double().abs()
    g = got.detach().cpu().double().reshape(ref.shape)
    bound = prop + _ulp16(ref.abs() + prop) + 1e-30
    excess = float(((g - ref).abs() / bound).max())
    rounded = ref.float().to(torch.bfloat16).double()
    den = rounded.norm(dim=-1)
    rel = torch.where(den > 0, (g - rounded).norm(dim=-1) / den.clamp_min(1e-300),
                      (g - rounded).norm(dim=-1))
    q99 = float(torch.quantile(rel, 0.99))
    print(f"{what}: max |err|/bound {excess:.3f}, row-norm rel err p99 {q99:.3e} "
          f"max {float(rel.max()):.3e}", flush=True)
    assert excess <= 1.0, f"{what}: an element exceeds its propagated bound ({excess:.3f}x)"
    assert q99 <= 2e-3, f"{what}: 99th percentile row-norm rel err {q99:.3e} > 2e-3"


@pytest.mark.parametrize("V", [4099, 8256])
@pytest.mark.parametrize("row_block", [64, 192, 4096])
def test_linear_logprobs_and_grads(device, V, row_block):
    print(f"[linear-logprobs] V={V} row_block={row_block}", flush=True)
    B, T, H = 8, 96, 256
    h, w, x, t, _old, _adv, _mask = _inputs(41, B, T, H, V, torch.bfloat16, device, row_block)
    hd = h.to(device).requires_grad_()
    wd = w.to(device).requires_grad_()
    lp = R.linear_token_logprobs(hd, wd, t.to(device), row_block=row_block)
    assert lp.dtype == torch.float32 and lp.shape == (B, T)
    lpo = o.token_logprobs(x, t, exact=True)
    err = (lp.detach().cpu().double() - lpo).abs()
    assert bool((err <= 1e-5 * lpo.abs() + 1e-7).all()), float(err.max())
    gw = torch.randn(B, T, generator=_gen(5))
    (lp * gw.to(device)).sum().backward()
    p = torch.softmax(x.double(), dim=-1)
    oh = torch.zeros_like(p).scatter_(-1, t[..., None], 1.0)
    # the reference's bf16 autograd rounds dlogits to bf16 before the linear
    # map's backward
    dl16 = (gw.double()[..., None] * (oh - p)).to(torch.bfloat16).double().reshape(-1, V)
    _product_check(hd.grad.reshape(-1, H), dl16, w, "dhidden", transpose=False)
    _product_check(wd.grad, dl16, h.reshape(-1, H), "dweight", transpose=True)


@pytest.mark.parametrize("objective", ["clipped", "sao", "sapo", "gspo", "gspo_token"])
@pytest.mark.parametrize("V,row_block", [(8256, 192), (4099, 64), (8256, 4096)])
def test_fused_linear_matches_oracle(device, objective, V, row_block):
    print(f"[fused-linear] objective={objective} V={V} row_block={row_block}", flush=True)
    B, T, H = 8, 96, 256
    h, w, x, t, old, adv, mask = _inputs(42, B, T, H, V, torch.bfloat16, device, row_block)
    kw = KW[objective]
    a = adv[:, 0].contiguous() if objective == "gspo" else adv
    hd = h.to(device).requires_grad_()
    wd = w.to(device).requires_grad_()
    d = lambda z: z.to(device)
    out, lp = R.fused_linear_policy_loss(hd, wd, d(t), d(old), d(a), d(mask), objective=objective,
                                         return_logprobs=True, row_block=row_block, **kw)
    out.loss.backward()
    kind = {"clipped": "ppo"}.get(objective, objective)
    out_o, lpo, dho, dwo = o.lm_head_step(kind, h, w, x, t, old, a, mask, exact=True, **kw)
    err = (lp.detach().cpu().double() - lpo).abs()
    assert bool((err <= 1e-5 * lpo.abs() + 1e-7).all()), float(err.max())
    scale = max(abs(out_o["loss"].item()), a.abs().mean().item())
    assert abs(out.loss.item() - out_o["loss"].item()) <= 2e-3 * scale, (
        out.loss.item(), out_o["loss"].item())
    assert hd.grad.dtype == torch.bfloat16 and wd.grad.dtype == torch.bfloat16
    dl16 = out_o["dlogits"].double().reshape(-1, V)
    _product_check(hd.grad.reshape(-1, H), dl16, w, "dhidden", transpose=False)
    _product_check(wd.grad, dl16, h.reshape(-1, H), "dweight", transpose=True)
    torch.testing.assert_close(dho.reshape(-1, H), dl16 @ w.double())  # the oracle's products


def test_fused_linear_float32(device):
    B, T, H, V = 8, 32, 128, 3001
    h, w, x, t, old, adv, mask = _inputs(43, B, T, H, V, torch.float32, device, 64)
    hd = h.to(device).requires_grad_()
    wd = w.to(device).requires_grad_()
    d = lambda z: z.to(device)
    out = R.fused_linear_policy_loss(hd, wd, d(t), d(old), d(adv), d(mask), row_block=64,
                                     **KW["clipped"])
    out.loss.backward()
    out_o, _lpo, dho, dwo = o.lm_head_step("ppo", h, w, x, t, old, adv, mask, exact=True,
                                           **KW["clipped"])
    scale = max(abs(out_o["loss"].item()), adv.abs().mean().item())
    assert abs(out.loss.item() - out_o["loss"].item()) <= 1e-5 * scale
    _rows_close(hd.grad.reshape(-1, H), dho.reshape(-1, H), 1e-5, "dhidden f32")
    _rows_close(wd.grad, dwo, 1e-5, "dweight f32")


def test_fused_linear_grad_scale_and_diagnostic_grads(device):
    """3 * loss scales both gradients; a loss that also differentiates a
    diagnostic (the KL term) takes the recomputing backward and equals the
    composition linear_token_logprobs -> clipped_policy_loss."""

    B, T, H, V = 8, 48, 128, 4104
    h, w, x, t, old, adv, mask = _inputs(44, B, T, H, V, torch.bfloat16, device, 128)
    d = lambda z: z.to(device)

    def run(fused, f):
        hd = d(h).requires_grad_()
        wd = d(w).requires_grad_()
        if fused:
            out = R.fused_linear_policy_loss(hd, wd, d(t), d(old), d(adv), d(mask), row_block=128,
                                             **KW["clipped"])
        else:
            lp = R.linear_token_logprobs(hd, wd, d(t), row_block=128)
            out = R.clipped_policy_loss(lp, d(old), d(adv), d(mask), **KW["clipped"])
        f(out).backward()
        return out, hd.grad, wd.grad

    o1, h1, w1 = run(True, lambda out: out.loss)
    o3, h3, w3 = run(True, lambda out: 3.0 * out.loss)
    torch.testing.assert_close(h3.float(), 3.0 * h1.float(), rtol=8e-3, atol=1e-6)
    torch.testing.assert_close(w3.float(), 3.0 * w1.float(), rtol=8e-3, atol=1e-6)
    _ok, hk, wk = run(True, lambda out: out.loss + 0.5 * out.approximate_kl)
    _oc, hc, wc = run(False, lambda out: out.loss + 0.5 * out.approximate_kl)
    _rows_close(hk.reshape(-1, H), hc.reshape(-1, H).double(), 4e-3, "dhidden with kl")
    _rows_close(wk, wc.double(), 4e-3, "dweight with kl")


def test_fused_linear_equals_logits_level_path(device):
    """The same row kernel as fused_policy_loss: log-probs bit-identical and
    the loss equal when fed the same block products."""

    B, T, H, V = 8, 64, 256, 8256
    h, w, x, t, old, adv, mask = _inputs(45, B, T, H, V, torch.bfloat16, device, 128)
    d = lambda z: z.to(device)
    out_l, lp_l = R.fused_linear_policy_loss(d(h), d(w).requires_grad_(), d(t), d(old), d(adv),
                                             d(mask), return_logprobs=True, row_block=128,
                                             **KW["clipped"])
    xd = d(x).requires_grad_()
    out_x, lp_x = R.fused_policy_loss(xd, d(t), d(old), d(adv), d(mask), return_logprobs=True,
                                      **KW["clipped"])
    assert torch.equal(lp_l, lp_x)
    torch.testing.assert_close(out_l.loss, out_x.loss, rtol=1e-6, atol=1e-9)
