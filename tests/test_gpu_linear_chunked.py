"""The chunked LM-head path beyond the tile path's shapes (MI355X): float32,
float16, bfloat16 and float64 weights, hidden sizes that are not multiples of
128 and above 1024 (Qwen3's 2048 and 4096), several row blocks per call, SFT
cross-entropy, evaluation without gradients, and gradients asked for one
operand only.

Oracle: the float64 chain (``o.lm_head_step``) on the logits the path
consumed, recorded by ``linear.record_logits`` and pinned to the exact
products: float32 within the accumulation's reach 6 sqrt(H) 2^-24 sum_k
|h_k w_vk|, 16-bit logits within one ulp of the exact product rounded to
nearest even plus that reach (at most 1e-3 of them on the other side of a
rounding midpoint), float64 within 1e-12 of sum_k |h_k w_vk| (the
reference's ``F.linear`` hands its log-softmax the same products,
rosetrainer/model.py:499,641).  Bars:

* log-probs within 1e-5 relative (+1e-6) of the oracle;
* the loss within 2e-3 of the terms' scale (1e-5 for float32 and float64);
* d hidden and d weight: 16-bit dtypes elementwise within twice the bound
  one-ulp deviations of the 16-bit dlogits move the product, plus one output
  ulp (float16 spacing floors at its subnormal step 2^-24); float32 and
  float64 row-norm-wise within 1e-5 and 1e-10 of the float64 product.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import roserlhf_oracle as o
from rosellm_amd import roserlhf as R
from rosellm_amd import rosetrainer as RT
from rosellm_amd.roserlhf import linear as LIN

from test_gpu_linear import _same_grads

pytestmark = pytest.mark.gpu

KW = {"clipped": dict(clip_low=0.2, clip_high=0.28), "gspo": dict(clip_low=3e-4, clip_high=4e-4),
      "sapo": dict(tau_positive=1.0, tau_negative=1.05)}
BITS = {torch.bfloat16: 8, torch.float16: 11, torch.float32: 24, torch.float64: 53}


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _ulp(v, dtype):
    m, e = torch.frexp(v.double())
    u = torch.ldexp(torch.ones_like(m), e - BITS[dtype])
    if dtype == torch.float16:
        u = torch.clamp(u, min=2.0 ** -24)
    return torch.where(v != 0, u, torch.zeros_like(u) + (2.0 ** -24 if dtype == torch.float16
                                                         else 0.0))


def _inputs(seed, B, T, H, V, dtype):
    g = _gen(seed)
    h = torch.randn(B, T, H, generator=g).to(dtype)
    w = (torch.randn(V, H, generator=g) * (2.0 / H ** 0.5)).to(dtype)
    x = h.double() @ w.double().t()
    t = torch.multinomial(torch.softmax(x, dim=-1).reshape(-1, V), 1, generator=g).reshape(B, T)
    lp = o.token_logprobs(x, t, exact=True).float()
    old = lp + torch.randn(B, T, generator=g) * 0.1
    lengths = torch.randint(1, T + 1, (B,), generator=g)
    mask = torch.arange(T)[None, :] < lengths[:, None]
    r = torch.randint(0, 2, (max(B // 4, 1), 4 if B >= 4 else B), generator=g).float()
    adv = o.group_standardize(r).reshape(-1)[:B, None].expand(B, T).contiguous()
    return h, w, x, t, old, adv, mask


def _consumed(rec, h, w, x, dtype):
    """(x_fwd, x_bwd) float64 [N, V]: the first and the last logits each token
    was formed with (record_logits), pinned to the exact products ``x``; rows
    never formed take the exact products in ``dtype``."""

    V = x.shape[-1]
    xr = x.reshape(-1, V)
    xd = xr if dtype == torch.float64 else xr.to(dtype).double()
    N = xr.shape[0]
    xf = torch.full_like(xd, float("nan"))
    xb = xf.clone()
    seen = torch.zeros(N, dtype=torch.bool)
    for rows, lg in rec.blocks:
        r, v = rows.cpu(), lg.cpu().double()
        first = ~seen[r]
        xf[r[first]] = v[first]
        xb[r] = v
        seen[r] = True
    H = h.shape[-1]
    mag = h.reshape(-1, H).double().abs() @ w.double().abs().t()
    reach = 6 * math.sqrt(H) * 2.0 ** -24 * mag  # float32 accumulation
    if dtype == torch.float32:
        tol = reach
    elif dtype == torch.float64:
        tol = 1e-12 * (1 + mag)
    else:
        tol = _ulp(xd.abs(), dtype) + reach
    for xc in (xf, xb):
        diff = (xc[seen] - xr[seen]).abs() if dtype in (torch.float32, torch.float64) else (
            xc[seen] - xd[seen]).abs()
        assert bool((diff <= tol[seen] + 1e-30).all()), f"a {dtype} logit off its bound"
        if dtype in (torch.bfloat16, torch.float16):
            off = float((diff > 0).double().mean())
            assert off <= 1e-3, f"{off:.2e} of the logits rounded to the other neighbour"
    xf = torch.where(torch.isnan(xf), xd, xf)
    xb = torch.where(torch.isnan(xb), xf, xb)
    return xf.view(x.shape), xb.view(x.shape)


def _logp_check(lp, xf, t):
    lpo = o.token_logprobs(xf, t, exact=True)
    err = (lp.detach().cpu().double() - lpo).abs()
    bad = err > 1e-5 * lpo.abs() + 1e-6
    assert not bool(bad.any()), f"log-probs: worst abs err {float(err.max()):.3e}"
    return lpo


def _dlogits(out_o, xf, xb, t, dtype):
    """The oracle's dlogits, re-formed for the tokens whose backward formed
    their logits again (another row block: GSPO) from those logits and the
    forward log-sum-exp, as the row kernel forms them; rounded to 16-bit
    dtypes as the reference's autograd rounds them."""

    V = xf.shape[-1]
    dl = out_o["dlogits"].reshape(-1, V).double().clone()
    xf2, xb2 = xf.reshape(-1, V), xb.reshape(-1, V)
    rows = torch.nonzero((xf2 != xb2).any(dim=1)).reshape(-1)
    if rows.numel():
        g = out_o["dloss_dlogp"].reshape(-1).double()[rows]
        ta = t.reshape(-1)[rows]
        lse = torch.logsumexp(xf2[rows], dim=1)
        lpf = xf2[rows].gather(1, ta[:, None]).squeeze(1) - lse
        d = -g[:, None] * torch.exp(xb2[rows] - lse[:, None])
        d.scatter_(1, ta[:, None], (-g * torch.expm1(lpf))[:, None])
        dl[rows] = d.to(dtype).double() if dtype in (torch.bfloat16, torch.float16) else d
    return dl


def _grad_check(got, dl, other, what, transpose, dtype):
    """got = dl @ other (transpose=False) or dl.T @ other; dl: the oracle's
    dlogits (rounded to ``dtype`` for 16-bit dtypes, as its chain does)."""

    dlw = dl.double()
    a = dlw.t() if transpose else dlw
    ref = a @ other.double()
    g = got.detach().cpu().double().reshape(ref.shape)
    if dtype in (torch.bfloat16, torch.float16):
        ua = _ulp(a.abs(), dtype)
        prop = ua @ other.double().abs()
        bound = 2.0 * prop + _ulp(ref.abs() + prop, dtype) + 1e-30
        excess = float(((g - ref).abs() / bound).max())
        print(f"{what}: max |err|/bound {excess:.3f}", flush=True)
        assert excess <= 1.0, f"{what}: an element exceeds its propagated bound ({excess:.3f}x)"
    else:
        tol = 1e-5 if dtype == torch.float32 else 1e-10
        den = ref.norm(dim=-1)
        rel = torch.where(den > 0, (g - ref).norm(dim=-1) / den.clamp_min(1e-300),
                          (g - ref).norm(dim=-1))
        print(f"{what}: max row-norm rel err {float(rel.max()):.3e}", flush=True)
        assert float(rel.max()) <= tol, what


@pytest.mark.parametrize("objective", ["clipped", "gspo"])
@pytest.mark.parametrize("dtype,H", [(torch.float32, 200), (torch.float32, 1024),
                                     (torch.float16, 200), (torch.bfloat16, 200),
                                     (torch.bfloat16, 2048), (torch.bfloat16, 4096),
                                     (torch.float64, 96)], ids=str)
def test_chunked_dtypes_hidden_sizes_and_row_blocks(device, dtype, H, objective):
    print(f"[chunked] dtype={dtype} H={H} objective={objective}", flush=True)
    B, T, V = 4, 29, 1031
    h, w, x, t, old, adv, mask = _inputs(60 + H, B, T, H, V, dtype)
    kw = KW[objective]
    a = adv[:, 0].contiguous() if objective == "gspo" else adv
    hd = h.to(device).requires_grad_()
    wd = w.to(device).requires_grad_()
    d = lambda z: z.to(device)  # noqa: E731
    # row blocks of 37 tokens: the 116 tokens (and their active subset) span
    # several blocks, the last one partial
    with LIN.record_logits() as rec:
        out, lp = R.fused_linear_policy_loss(hd, wd, d(t), d(old), d(a), d(mask),
                                             objective=objective, return_logprobs=True,
                                             row_block=37, **kw)
        out.loss.backward()
    assert hd.grad.dtype == dtype and wd.grad.dtype == dtype
    xf, xb = _consumed(rec, h, w, x, dtype)
    _logp_check(lp, xf, t)
    kind = {"clipped": "ppo"}.get(objective, objective)
    xi = xf if dtype == torch.float64 else xf.to(dtype)
    out_o, _lpo, _dho, _dwo = o.lm_head_step(kind, h, w, xi, t, old, a, mask, exact=True, **kw)
    out_o["dlogits"] = _dlogits(out_o, xf, xb, t, dtype)
    scale = max(abs(out_o["loss"].item()), a.abs().mean().item())
    rtol = 2e-3 if dtype in (torch.bfloat16, torch.float16) else 1e-5
    assert abs(out.loss.item() - out_o["loss"].item()) <= rtol * scale, (
        out.loss.item(), out_o["loss"].item())
    dl = out_o["dlogits"].reshape(-1, V)
    _grad_check(hd.grad.reshape(-1, H), dl, w, "dhidden", False, dtype)
    _grad_check(wd.grad, dl, h.reshape(-1, H), "dweight", True, dtype)


@pytest.mark.parametrize("dtype,H", [(torch.float32, 200), (torch.bfloat16, 2048)], ids=str)
def test_chunked_cross_entropy(device, dtype, H):
    """SFT loss of the final hidden states (rosetrainer/model.py:641-649)
    through the chunked LM head, ignored labels included."""

    print(f"[chunked sft] dtype={dtype} H={H}", flush=True)
    g = _gen(70)
    B, T, V = 3, 41, 777
    h = torch.randn(B, T, H, generator=g).to(dtype)
    w = (torch.randn(V, H, generator=g) * (2.0 / H ** 0.5)).to(dtype)
    y = torch.randint(0, V, (B, T), generator=g)
    y[torch.rand(B, T, generator=g) < 0.2] = -100
    hd = h.to(device).requires_grad_()
    wd = w.to(device).requires_grad_()
    with LIN.record_logits() as rec:
        loss = RT.linear_causal_lm_loss(hd, wd, y.to(device), row_block=50)
        loss.backward()
    hs = h[:, :-1].contiguous()
    xf, _xb = _consumed(rec, hs, w, hs.double() @ w.double().t(), dtype)
    want, dl = o.sft_step(xf.to(dtype) if dtype != torch.float64 else xf, y[:, 1:],
                          causal=False, exact=True)
    assert abs(loss.item() - want.item()) <= 1e-5 * abs(want.item())
    assert bool((hd.grad[:, -1] == 0).all())
    dl = dl.reshape(-1, V)
    _grad_check(hd.grad[:, :-1].reshape(-1, H), dl, w, "dhidden", False, dtype)
    _grad_check(wd.grad, dl, hs.reshape(-1, H), "dweight", True, dtype)


def test_chunked_without_grad_and_one_sided_grads(device):
    """Evaluation (no gradients: every token takes the log-prob pass) gives the
    training step's loss; gradients asked for the weight only, or the hidden
    states only, equal those of the two-sided call."""

    B, T, H, V = 4, 50, 192, 2049
    h, w, _x, t, old, adv, mask = _inputs(71, B, T, H, V, torch.bfloat16)
    d = lambda z: z.to(device)  # noqa: E731
    kw = KW["clipped"]

    def run(gh, gw):
        hd = d(h).requires_grad_(gh)
        wd = d(w).requires_grad_(gw)
        out = R.fused_linear_policy_loss(hd, wd, d(t), d(old), d(adv), d(mask), row_block=64,
                                         **kw)
        if gh or gw:
            out.loss.backward()
        return out.loss.detach(), hd.grad, wd.grad

    with torch.no_grad():
        l_eval, _, _ = run(False, False)
    l_both, gh_both, gw_both = run(True, True)
    l_w, gh_w, gw_w = run(False, True)
    l_h, gh_h, gw_h = run(True, False)
    torch.testing.assert_close(l_eval, l_both, rtol=1e-6, atol=1e-7)
    assert gh_w is None and gw_h is None
    assert torch.equal(l_w, l_both) and torch.equal(l_h, l_both)
    _same_grads(gw_w, gw_both, "chunked", "d weight alone")
    _same_grads(gh_h, gh_both, "chunked", "d hidden alone")


@pytest.mark.parametrize("objective", ["clipped", "sapo"])
def test_chunked_upstream_scale(device, objective):
    """A loss scaled by 3 (float32 weights: the stored gradients are rescaled
    on the device) gives 3x the gradients."""

    B, T, H, V = 4, 40, 136, 1500
    h, w, _x, t, old, adv, mask = _inputs(72, B, T, H, V, torch.float32)
    d = lambda z: z.to(device)  # noqa: E731

    def run(f):
        hd = d(h).requires_grad_()
        wd = d(w).requires_grad_()
        out = R.fused_linear_policy_loss(hd, wd, d(t), d(old), d(adv), d(mask),
                                         objective=objective, row_block=33, **KW[objective])
        f(out.loss).backward()
        return hd.grad, wd.grad

    h1, w1 = run(lambda z: z)
    h3, w3 = run(lambda z: 3.0 * z)
    # float32: within float32 accumulation (the GEMM's reduction order may
    # vary from run to run), row-norm-wise
    for a, b, what in ((h3, 3.0 * h1, "d hidden"), (w3, 3.0 * w1, "d weight")):
        num, den = (a - b).norm(dim=-1), b.norm(dim=-1)
        worst = float(torch.where(den > 0, num / den.clamp_min(1e-30), num).max())
        assert worst <= 1e-5, f"{what}: row-norm rel diff {worst:.3e}"


@pytest.mark.parametrize("rows,cols,pad,offset", [(151936 // 16, 1024, 0, 0), (1000, 1030, 0, 0),
                                                  (777, 129, 24, 0), (300, 64, 8, 3),
                                                  (65, 1, 0, 0), (1, 70, 0, 1)])
def test_transpose16_is_exact(device, rows, cols, pad, offset):
    """rrl_transpose16 (the weight's [H, V] copy for the d hidden GEMM) against
    torch's transpose, bit for bit: partial 64 x 64 tiles on both sides,
    padded source rows, and sources off 16-byte alignment (the element-wise
    path)."""

    from rosellm_amd import _native as nat

    g = _gen(rows * 3 + cols)
    base = torch.randn(rows * (cols + pad) + offset, generator=g).to(torch.bfloat16).to(device)
    src = base[offset:].view(rows, cols + pad)[:, :cols]
    dst = torch.full((cols, rows + 8), float("nan"), dtype=torch.bfloat16, device=device)
    nat.call("rrl_transpose16", src.data_ptr(), rows, cols, src.stride(0), dst.data_ptr(),
             dst.stride(0), nat.stream_ptr(device))
    torch.cuda.synchronize()
    assert torch.equal(dst[:, :rows].view(torch.int16), src.t().contiguous().view(torch.int16))
    assert torch.isnan(dst[:, rows:].float()).all(), "a store landed past the rows"
