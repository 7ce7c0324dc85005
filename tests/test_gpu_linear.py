"""Matrix-core LM head (config 5) vs the CPU oracle on identical seeded inputs.

The oracle runs the whole chain exactly: the float64 product of the bf16
hidden states and weight (``hidden.double() @ weight.double().T``), then
``lm_head_step`` in float64, whose dlogits are rounded to bf16 before the two
backward products, as the reference's bf16 autograd rounds them.  Bars:

* log-probs within 1e-5 relative (+1e-6 absolute) of the float64 oracle: the
  kernels accumulate the 16-bit products in float32;
* the loss within 2e-3 of the objective's term scale (bf16 inputs);
* d hidden and d weight (bf16): every element within twice what one-ulp
  deviations of the bf16 dlogits can move the product (``ulp(dlogits16) @
  |W|``, resp. ``ulp(dlogits16).T @ |hidden|``) plus one ulp of the output,
  around the float64 product of the correctly rounded dlogits.  The kernels
  round the softmax weight p (forward) or g (onehot - p) (dW pass) to bf16
  where the reference rounds g (onehot - p): each is within one ulp of the
  reference's value.  Row-wise against the exact product: every row within
  2^-7 (one bf16 ulp) norm-wise, and the 99th percentile within 2e-3 or
  1.25x that of the reference's own bf16 chain (bf16 dlogits, product
  rounded to bf16), whichever is larger.

Both implementations run every test that applies to them.  ``impl="tiles"``
(the hand-written kernels, which never round a logit) is held to the exact
float64 chain.  ``impl="chunked"`` forms each row block's logits with a
16-bit GEMM, rounded to bf16 as the reference's ``F.linear`` rounds them, so
its oracle is the same float64 chain run on the exact products rounded to
bf16 (``o.lm_head_step``'s ``logits`` argument): the log-probs within 1e-5
relative plus one bf16 ulp of the target logit and one of the row's largest
logit (the GEMM accumulates in float32, so a product within ~1e-6 of a bf16
rounding midpoint may round the other way), the rest as above.
"""

from __future__ import annotations

import contextlib
import dataclasses
import math

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


def _inputs(seed, B, T, H, V, w_scale=None, hot=0.0):
    """bf16 hidden ~ N(0, 1), weight ~ N(0, w_scale); the exact float64 logits;
    targets sampled from the softmax (``hot``: that fraction of tokens gets
    the arg-max as target, p_target near 1 when the weight is sharp)."""

    g = _gen(seed)
    h = torch.randn(B, T, H, generator=g).to(torch.bfloat16)
    ws = (2.0 / H ** 0.5) if w_scale is None else w_scale
    w = (torch.randn(V, H, generator=g) * ws).to(torch.bfloat16)
    x = h.double() @ w.double().t()
    probs = torch.softmax(x, dim=-1)
    t = torch.multinomial(probs.reshape(-1, V), 1, generator=g).reshape(B, T)
    if hot > 0:
        pick = torch.rand(B, T, generator=g) < hot
        t = torch.where(pick, x.argmax(dim=-1), t)
    lp = o.token_logprobs(x, t, exact=True).float()
    old = lp + torch.randn(B, T, generator=g) * 0.1
    lengths = torch.randint(1, T + 1, (B,), generator=g)
    mask = torch.arange(T)[None, :] < lengths[:, None]
    r = torch.randint(0, 2, (max(B // 4, 1), 4 if B >= 4 else B), generator=g).float()
    adv = o.group_standardize(r).reshape(-1)[:B, None].expand(B, T).contiguous()
    return h, w, x, t, old, adv, mask


def _ulp16(v):
    """bf16 unit in the last place of each (bf16-representable) value."""

    m, e = torch.frexp(v.double())
    return torch.where(v != 0, torch.ldexp(torch.ones_like(m), e - 8), torch.zeros_like(m))


def _product_check(got, dl, other, what, transpose, factor=2.0):
    """got: the kernel's d hidden (transpose=False: dl @ other) or d weight
    (transpose=True: dl.T @ other); dl: the exact dlogits [rows, V] (float64).

    Elementwise: within ``factor`` times the propagated one-ulp bound of the
    bf16 dlogits the reference's autograd forms (plus one output ulp) around
    the float64 product of those rounded dlogits.  Row-wise: 99% of the rows
    within 2e-3 norm-wise of the exact product (bf16's own precision: the
    kernels keep the target entry's 1 - p exact where the reference rounds
    it).  Every row within one bf16 ulp (2^-7) norm-wise."""

    dl16 = dl.to(torch.bfloat16).double()
    a16 = dl16.t() if transpose else dl16
    ref = a16 @ other.double()
    prop = (_ulp16(dl16).t() if transpose else _ulp16(dl16)) @ other.double().abs()
    g = got.detach().cpu().double().reshape(ref.shape)
    bound = factor * prop + _ulp16(ref.abs() + prop) + 1e-30
    excess = float(((g - ref).abs() / bound).max())
    exact = (dl.t() if transpose else dl) @ other.double()
    den = exact.norm(dim=-1)

    def rowrel(v):
        return torch.where(den > 0, (v - exact).norm(dim=-1) / den.clamp_min(1e-300),
                           (v - exact).norm(dim=-1))

    rel = rowrel(g)
    # the reference's own chain: bf16 dlogits, their product rounded to bf16
    rel_ref = rowrel(ref.float().to(torch.bfloat16).double())
    q99, q99_ref = float(torch.quantile(rel, 0.99)), float(torch.quantile(rel_ref, 0.99))
    print(f"{what}: max |err|/bound {excess:.3f}; row-norm rel err vs exact: p99 {q99:.3e} "
          f"max {float(rel.max()):.3e} (the reference's bf16 chain: p99 {q99_ref:.3e} max "
          f"{float(rel_ref.max()):.3e})", flush=True)
    assert excess <= 1.0, f"{what}: an element exceeds its propagated bound ({excess:.3f}x)"
    assert float(rel.max()) <= 2.0 ** -7, f"{what}: a row beyond bf16 precision"
    assert q99 <= max(2e-3, 1.25 * q99_ref), (
        f"{what}: 99th percentile row-norm rel err {q99:.3e} (reference chain {q99_ref:.3e})")


def _exact_dlogits(x, t, g):
    """g (onehot - softmax(x)) in float64 with the target entry formed as
    g * sigmoid(logsumexp_{v != a}(x_v - x_a)) = g (1 - p_a), which keeps its
    relative precision as p_a -> 1 (1 - p_a in float64 rounds to 0 once the
    gap exceeds ~37)."""

    V = x.shape[-1]
    x2, t2, g2 = x.reshape(-1, V), t.reshape(-1), g.reshape(-1).double()
    p = torch.softmax(x2, dim=-1)
    dl = -g2[:, None] * p
    xa = x2.gather(1, t2[:, None])
    rest = (x2 - xa).scatter(1, t2[:, None], float("-inf"))
    one_minus = torch.sigmoid(torch.logsumexp(rest, dim=-1))
    dl.scatter_(1, t2[:, None], (g2 * one_minus)[:, None])
    return dl


def _logp_check(lp, lpo, scale=None):
    """Within 1e-5 relative plus the float32 accumulation error of logits of
    magnitude ``scale`` (1e-7 of it, at least 1e-6 absolute)."""

    err = (lp.detach().cpu().double() - lpo).abs()
    floor = 1e-6 if scale is None else max(1e-6, 1e-7 * float(scale))
    bad = err > 1e-5 * lpo.abs() + floor
    assert not bool(bad.any()), f"log-probs: worst abs err {float(err.max()):.3e}"


IMPLS = ["tiles", "chunked"]


def _same_grads(a, b, impl, what, tol=2.0 ** -7):
    """Gradients of two separate runs: bit-identical on the tile path; on the
    chunked path within two bf16 roundings row-norm-wise (the GEMM library
    may split d hidden's long reduction over the vocabulary across workgroups
    and combine the float32 partial sums in a run-dependent order, which can
    round an element to the neighbouring bf16 value)."""

    if impl == "tiles":
        assert torch.equal(a, b), what
        return
    x, y = a.float().reshape(-1, a.shape[-1]), b.float().reshape(-1, b.shape[-1])
    num, den = (x - y).norm(dim=-1), y.norm(dim=-1)
    worst = float(torch.where(den > 0, num / den.clamp_min(1e-30), num).max())
    print(f"{what}: worst row-norm rel diff {worst:.3e}", flush=True)
    assert worst <= tol, f"{what}: row-norm rel diff {worst:.3e}"


def _tap(impl):
    """Records the logits the chunked path consumes (linear.record_logits);
    nothing to record on the tile path."""

    return LIN.record_logits() if impl == "chunked" else contextlib.nullcontext()


def _consumed(impl, rec, x, h, w):
    """(x_fwd, x_bwd): the float64 logits ``impl`` formed each token's
    log-prob from, and those its backward formed the token's dlogits from.
    The tile path's are the exact products.  The chunked path's are its
    GEMM's bf16 outputs as record_logits kept them, pinned here to the exact
    products ``x`` of ``h`` and ``w`` rounded to nearest even: every one
    within one bf16 ulp of that plus the float32 accumulation's reach
    (6 sqrt(H) 2^-24 sum_k |h_k w_vk|), at most 1e-3 of them on the other
    side of a rounding midpoint.  Rows the chunked path never formed
    (skip_masked_rows) take the rounded products."""

    if impl == "tiles":
        return x, x
    V = x.shape[-1]
    H = h.shape[-1]
    x16 = x.reshape(-1, V).to(torch.bfloat16).double()
    reach = 6 * math.sqrt(H) * 2.0 ** -24 * (h.reshape(-1, H).double().abs()
                                            @ w.double().abs().t())
    N = x16.shape[0]
    xf = torch.full_like(x16, float("nan"))
    xb = xf.clone()
    seen = torch.zeros(N, dtype=torch.bool)
    for rows, lg in rec.blocks:
        r, v = rows.cpu(), lg.cpu().double()
        first = ~seen[r]
        xf[r[first]] = v[first]
        xb[r] = v
        seen[r] = True
    for xc in (xf, xb):
        ok = seen
        diff = (xc[ok] - x16[ok]).abs()
        assert bool((diff <= _ulp16(x16[ok].abs()) + reach[ok] + 1e-30).all()), (
            "a logit beyond one ulp and the accumulation's reach")
        off = float((diff > 0).double().mean()) if diff.numel() else 0.0
        assert off <= 1e-3, f"{off:.2e} of the logits rounded to the other neighbour"
    xf = torch.where(torch.isnan(xf), x16, xf)
    xb = torch.where(torch.isnan(xb), xf, xb)
    return xf.view(x.shape), xb.view(x.shape)


def _oracle_step(impl, kind, h, w, x, t, old, a, mask, rec, **kw):
    """o.lm_head_step in float64 on the logits ``impl`` consumed.  A chunked
    backward that formed a token's logits again (GSPO: another row block)
    gets that token's dlogits from those logits and its forward log-sum-exp,
    as the row kernel forms them."""

    xf, xb = _consumed(impl, rec, x, h, w)
    out_o, _lpo, _dho, _dwo = o.lm_head_step(kind, h, w, xf, t, old, a, mask, exact=True, **kw)
    if impl == "chunked" and not torch.equal(xf, xb):
        V = x.shape[-1]
        xf2, xb2 = xf.reshape(-1, V), xb.reshape(-1, V)
        rows = torch.nonzero((xf2 != xb2).any(dim=1)).reshape(-1)
        g = out_o["dloss_dlogp"].reshape(-1).double()[rows]
        ta = t.reshape(-1)[rows]
        lse = torch.logsumexp(xf2[rows], dim=1)
        lpf = xf2[rows].gather(1, ta[:, None]).squeeze(1) - lse
        d = -g[:, None] * torch.exp(xb2[rows] - lse[:, None])
        d.scatter_(1, ta[:, None], (-g * torch.expm1(lpf))[:, None])
        dl = out_o["dlogits"].reshape(-1, V).double().clone()
        dl[rows] = d
        out_o["dlogits"] = dl.view(x.shape)
    return out_o


def _logp_check_impl(impl, lp, x, t, rec, h, w, scale=None):
    """The log-probs of ``impl`` against the float64 oracle on the logits it
    consumed, within 1e-5 relative (``_logp_check``)."""

    xf, _xb = _consumed(impl, rec, x, h, w)
    lpo = o.token_logprobs(xf, t, exact=True)
    _logp_check(lp, lpo, scale)
    return lpo


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("H,V", [(256, 4099), (1024, 8256), (384, 1000), (128, 33),
                                 (768, 2050), (896, 301), (512, 1), (128, 19201)])
def test_linear_logprobs_and_grads(device, H, V, impl):
    """log-probs and, for a random upstream gradient, d hidden and d weight,
    across hidden sizes (every instantiated one is a multiple of 128 up to
    1024), vocabularies that are not tile multiples, and token counts that
    are not 64-row block multiples.  V = 19201 has 301 weight blocks: on a
    256-CU device the dW pass splits the last 45 over token ranges and sums
    their partial rows."""

    print(f"[linear-logprobs] impl={impl} H={H} V={V}", flush=True)
    B, T = 3, 37
    h, w, x, t, _old, _adv, _mask = _inputs(41, B, T, H, V)
    hd = h.to(device).requires_grad_()
    wd = w.to(device).requires_grad_()
    gw = torch.randn(B, T, generator=_gen(5))
    with _tap(impl) as rec:
        lp = R.linear_token_logprobs(hd, wd, t.to(device), impl=impl)
        (lp * gw.to(device)).sum().backward()
    assert lp.dtype == torch.float32 and lp.shape == (B, T)
    _logp_check_impl(impl, lp, x, t, rec, h, w)
    _xf, xb = _consumed(impl, rec, x, h, w)
    lse = torch.logsumexp(_xf, dim=-1, keepdim=True)
    p = torch.exp(xb - lse)
    oh = torch.zeros_like(p).scatter_(-1, t[..., None], 1.0)
    dl = (gw.double()[..., None] * (oh - p)).reshape(-1, V)
    assert hd.grad.dtype == torch.bfloat16 and wd.grad.dtype == torch.bfloat16
    _product_check(hd.grad.reshape(-1, H), dl, w, "dhidden", transpose=False)
    _product_check(wd.grad, dl, h.reshape(-1, H), "dweight", transpose=True)


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("objective", ["clipped", "sao", "sapo", "gspo", "gspo_token"])
def test_fused_linear_matches_oracle(device, objective, impl):
    print(f"[fused-linear] impl={impl} objective={objective}", flush=True)
    B, T, H, V = 8, 96, 256, 8256
    h, w, x, t, old, adv, mask = _inputs(42, B, T, H, V)
    kw = KW[objective]
    a = adv[:, 0].contiguous() if objective == "gspo" else adv
    hd = h.to(device).requires_grad_()
    wd = w.to(device).requires_grad_()
    d = lambda z: z.to(device)  # noqa: E731
    with _tap(impl) as rec:
        out, lp = R.fused_linear_policy_loss(hd, wd, d(t), d(old), d(a), d(mask),
                                             objective=objective, return_logprobs=True,
                                             impl=impl, **kw)
        out.loss.backward()
    kind = {"clipped": "ppo"}.get(objective, objective)
    # the whole chain in float64 on the logits the implementation consumed
    _logp_check_impl(impl, lp, x, t, rec, h, w)
    out_o = _oracle_step(impl, kind, h, w, x, t, old, a, mask, rec, **kw)
    scale = max(abs(out_o["loss"].item()), a.abs().mean().item())
    assert abs(out.loss.item() - out_o["loss"].item()) <= 2e-3 * scale, (
        out.loss.item(), out_o["loss"].item())
    dl = out_o["dlogits"].double().reshape(-1, V)  # float64 on the consumed logits
    _product_check(hd.grad.reshape(-1, H), dl, w, "dhidden", transpose=False)
    _product_check(wd.grad, dl, h.reshape(-1, H), "dweight", transpose=True)


@pytest.mark.parametrize("impl", IMPLS)
def test_dominant_targets_keep_precision(device, impl):
    """Sharp weights and arg-max targets: p_target -> 1, where 1 - p_target
    must come from expm1(logp), not from 1 - p."""

    B, T, H, V = 4, 64, 256, 4096
    h, w, x, t, _old, _adv, _mask = _inputs(43, B, T, H, V, w_scale=2.0, hot=0.8)
    hd = h.to(device).requires_grad_()
    wd = w.to(device).requires_grad_()
    gw = torch.randn(B, T, generator=_gen(6))
    with _tap(impl) as rec:
        lp = R.linear_token_logprobs(hd, wd, t.to(device), impl=impl)
        (lp * gw.to(device)).sum().backward()
    lpo = _logp_check_impl(impl, lp, x, t, rec, h, w, scale=x.abs().max())  # logits reach ~100 here
    print(f"dominant: min p_target {float(lpo.exp().min()):.3e}, "
          f"max p_target {float(lpo.exp().max()):.9f}", flush=True)
    assert float(lpo.exp().max()) > 0.999
    xf, xb = _consumed(impl, rec, x, h, w)
    assert torch.equal(xf, xb)  # one formation per token
    dl = _exact_dlogits(xf, t, gw)
    _product_check(hd.grad.reshape(-1, H), dl, w, "dhidden", transpose=False)
    _product_check(wd.grad, dl, h.reshape(-1, H), "dweight", transpose=True)


@pytest.mark.parametrize("impl", IMPLS)
def test_logits_beyond_the_reference_range_rerun(device, impl):
    """One weight row that gives some tokens logits far above their first
    tile's maximum (beyond the tile path's fixed reference range): the tile
    path reruns around the exact log-sum-exp; both paths match the oracle."""

    B, T, H, V = 2, 64, 256, 2048
    h, w, _x, _t, _old, _adv, _mask = _inputs(44, B, T, H, V)
    w[1000] = (h[0, 0].float() * 0.6).to(torch.bfloat16)  # logit ~ 0.6 * |h|^2 ~ 150 for token 0
    x = h.double() @ w.double().t()
    t = torch.randint(0, V, (B, T), generator=_gen(7))
    first = x[..., :32].max(dim=-1).values
    assert float((x.max(dim=-1).values - first).max()) > 100.0
    hd = h.to(device).requires_grad_()
    wd = w.to(device).requires_grad_()
    gw = torch.randn(B, T, generator=_gen(8))
    with _tap(impl) as rec:
        lp = R.linear_token_logprobs(hd, wd, t.to(device), impl=impl)
        (lp * gw.to(device)).sum().backward()
    _logp_check_impl(impl, lp, x, t, rec, h, w, scale=x.abs().max())
    xf, xb = _consumed(impl, rec, x, h, w)
    p = torch.exp(xb - torch.logsumexp(xf, dim=-1, keepdim=True))
    oh = torch.zeros_like(p).scatter_(-1, t[..., None], 1.0)
    dl = (gw.double()[..., None] * (oh - p)).reshape(-1, V)
    _product_check(hd.grad.reshape(-1, H), dl, w, "dhidden", transpose=False)
    _product_check(wd.grad, dl, h.reshape(-1, H), "dweight", transpose=True)


@pytest.mark.parametrize("impl", IMPLS)
def test_range_rerun_with_skipped_blocks(device, impl):
    """The rerun around the exact log-sum-exp (a logit far beyond the single
    pass's reference range) with skip_masked_rows: the rerun keeps the
    skipped blocks out too, and the loss and both gradients equal the full
    computation's bit for bit."""

    B, T, H, V = 4, 128, 256, 2048
    h, w, _x, t, old, adv, _mask = _inputs(45, B, T, H, V)
    w[1000] = (h[0, 0].float() * 0.6).to(torch.bfloat16)  # token (0, 0): logit ~ 150
    x = h.double() @ w.double().t()
    assert float(x[0, 0].max() - x[0, 0, :32].max()) > 100.0
    lengths = torch.tensor([128, 0, 64, 5])  # blocks of 64: 2 live, 2 masked, 1 + 1, 1 + 1
    mask = torch.arange(T)[None, :] < lengths[:, None]
    d = lambda z: z.to(device)  # noqa: E731
    res = []
    for skip in (False, True):
        hd = h.to(device).requires_grad_()
        wd = w.to(device).requires_grad_()
        with _tap(impl) as rec:
            out = R.fused_linear_policy_loss(hd, wd, d(t), d(old), d(adv), d(mask),
                                             objective="clipped", skip_masked_rows=skip,
                                             impl=impl, **KW["clipped"])
            out.loss.backward()
        res.append((out.loss, hd.grad, wd.grad))
        if not skip:
            rec0 = rec
    (l0, h0, w0), (l1, h1, w1) = res
    assert torch.equal(l0, l1)
    _same_grads(h0, h1, impl, "d hidden")
    _same_grads(w0, w1, impl, "d weight")
    out_o = _oracle_step(impl, "ppo", h, w, x, t, old, adv, mask, rec0, **KW["clipped"])
    scale = max(abs(out_o["loss"].item()), adv.abs().mean().item())
    assert abs(l0.item() - out_o["loss"].item()) <= 2e-3 * scale


@pytest.mark.parametrize("H,V,B,T,hot", [(1024, 8256, 3, 67, 0.0), (128, 33, 2, 32, 0.0),
                                         (384, 1000, 2, 129, 0.0), (768, 2050, 2, 1, 0.0),
                                         (256, 4096, 4, 64, 0.8)])
@pytest.mark.parametrize("impl", IMPLS)
def test_logprobs_without_grad_lse_pass(device, H, V, B, T, hot, impl):
    """Without a gradient the log-probs come from the log-sum-exp-only kernel
    (128 tokens per workgroup: token counts that fill one, two or three
    64-token halves of it, vocabularies off the 32-column tile, targets that
    dominate their row)."""

    print(f"[lse-pass] H={H} V={V} N={B * T} hot={hot}", flush=True)
    h, w, x, t, _old, _adv, _mask = _inputs(47, B, T, H, V, w_scale=2.0 if hot else None,
                                           hot=hot)
    with torch.no_grad(), _tap(impl) as rec:
        lp = R.linear_token_logprobs(h.to(device), w.to(device), t.to(device), impl=impl)
    assert lp.dtype == torch.float32 and lp.shape == (B, T)
    _logp_check_impl(impl, lp, x, t, rec, h, w, scale=x.abs().max())


@pytest.mark.parametrize("impl", IMPLS)
def test_fused_linear_masked_blocks_interleaved(device, impl):
    """Masks whose fully masked 64-token blocks alternate with needed ones:
    the needed blocks take the obar pass, the others the log-sum-exp pass
    (two per workgroup, not adjacent in memory), and every log-prob, the loss
    and both gradients match the oracle."""

    B, T, H, V = 8, 192, 256, 4099
    h, w, x, t, old, adv, _mask = _inputs(48, B, T, H, V)
    lengths = torch.tensor([64, 192, 0, 130, 1, 65, 128, 0])
    mask = torch.arange(T)[None, :] < lengths[:, None]
    blocks = mask.reshape(-1, 64).any(dim=1)
    assert bool(blocks.any()) and not bool(blocks.all())
    kw = KW["clipped"]
    hd = h.to(device).requires_grad_()
    wd = w.to(device).requires_grad_()
    d = lambda z: z.to(device)  # noqa: E731
    with _tap(impl) as rec:
        out, lp = R.fused_linear_policy_loss(hd, wd, d(t), d(old), d(adv), d(mask),
                                             objective="clipped", return_logprobs=True,
                                             impl=impl, **kw)
        out.loss.backward()
    _logp_check_impl(impl, lp, x, t, rec, h, w)
    out_o = _oracle_step(impl, "ppo", h, w, x, t, old, adv, mask, rec, **kw)
    scale = max(abs(out_o["loss"].item()), adv.abs().mean().item())
    assert abs(out.loss.item() - out_o["loss"].item()) <= 2e-3 * scale
    dl = out_o["dlogits"].double().reshape(-1, V)
    _product_check(hd.grad.reshape(-1, H), dl, w, "dhidden", transpose=False)
    _product_check(wd.grad, dl, h.reshape(-1, H), "dweight", transpose=True)
    assert bool((hd.grad.reshape(-1, H)[~mask.reshape(-1).to(device)] == 0).all())


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("objective", ["clipped", "gspo", "sapo"])
def test_fused_linear_skip_masked_rows(device, objective, impl):
    """skip_masked_rows=True leaves out the 64-token blocks whose tokens are
    all masked: the loss, its diagnostics and both gradients are bit-identical
    to the full computation (a masked token's term is multiplied by 0)."""

    B, T, H, V = 8, 192, 256, 4099
    h, w, x, t, old, adv, _mask = _inputs(49, B, T, H, V)
    lengths = torch.tensor([64, 192, 0, 130, 1, 65, 128, 0])
    mask = torch.arange(T)[None, :] < lengths[:, None]
    if objective == "gspo":
        adv = adv[:, 0].contiguous()
    if objective in ("gspo", "sapo"):
        mask[2, 0] = mask[7, 0] = True  # per-sequence means need a token in every sequence
    d = lambda z: z.to(device)  # noqa: E731
    res = []
    for skip in (False, True):
        hd = h.to(device).requires_grad_()
        wd = w.to(device).requires_grad_()
        out = R.fused_linear_policy_loss(hd, wd, d(t), d(old), d(adv), d(mask),
                                         objective=objective, skip_masked_rows=skip,
                                         impl=impl, **KW[objective])
        out.loss.backward()
        res.append((out, hd.grad, wd.grad))
    (o0, h0, w0), (o1, h1, w1) = res
    for f in dataclasses.fields(o0):
        a, b = getattr(o0, f.name), getattr(o1, f.name)
        if isinstance(a, torch.Tensor):
            assert torch.equal(a, b), f.name
    _same_grads(h0, h1, impl, "d hidden")
    _same_grads(w0, w1, impl, "d weight")


def test_lm_head_fwd_blocks_needing_nothing(device):
    """The forward's per-token need values through the C ABI: a block whose
    64 tokens are all 2 gets lse = logp = 0 without being computed; a block
    with a 1 takes the obar pass and one with only 0s and 2s the
    log-sum-exp pass, both giving every token of the block its lse and logp
    (those of an obar-less call, within float32 rounding of the two passes)."""

    from rosellm_amd import _native as nat

    N, H, V = 640, 256, 4099
    h, w, _x, t, *_ = _inputs(50, 2, N // 2, H, V)
    hd, wd = h.reshape(N, H).to(device), w.to(device)
    t32 = t.reshape(N).to(torch.int32).to(device)
    # blocks: obar / lse / skip / obar / skip / lse / skip / skip / lse / obar
    kinds = [1, 0, 2, 1, 2, 0, 2, 2, 0, 1]
    need = torch.full((N,), 2, dtype=torch.uint8)
    for b, k in enumerate(kinds):
        if k == 1:
            need[64 * b + 5] = 1  # one token needs obar, the rest nothing
        elif k == 0:
            need[64 * b:64 * b + 64:7] = 0  # some need log-probs, the rest nothing
    need_d = need.to(device)
    st = nat.new_status(device)
    dt = nat.dtype_code(torch.bfloat16)
    s = nat.stream_ptr(device)
    ref_lse = torch.empty(N, device=device)
    ref_lp = torch.empty(N, device=device)
    nat.call("rrl_lm_head_fwd", hd.data_ptr(), wd.data_ptr(), dt, N, H, V, H, H, t32.data_ptr(),
             None, None, ref_lse.data_ptr(), ref_lp.data_ptr(), None, H, None, st.data_ptr(), s)
    lse = torch.full((N,), float("nan"), device=device)
    lp = torch.full((N,), float("nan"), device=device)
    obar = torch.empty(N, H, device=device)
    ws = torch.empty(nat.lib().rrl_lm_head_fwd_workspace_bytes(N), dtype=torch.uint8,
                     device=device)
    nat.call("rrl_lm_head_fwd", hd.data_ptr(), wd.data_ptr(), dt, N, H, V, H, H, t32.data_ptr(),
             need_d.data_ptr(), None, lse.data_ptr(), lp.data_ptr(), obar.data_ptr(), H,
             ws.data_ptr(), st.data_ptr(), s)
    assert nat.read_status(st) == 0
    order = ws[:4 * (len(kinds) + 2)].view(torch.int32).cpu().tolist()
    # obar blocks, then log-prob-only blocks, then the rest; then the counts
    assert order == [0, 3, 9, 1, 5, 8, 2, 4, 6, 7, 3, 6]
    for b, k in enumerate(kinds):
        sl = slice(64 * b, 64 * b + 64)
        if k == 2:
            assert bool((lse[sl] == 0).all()) and bool((lp[sl] == 0).all()), b
        else:
            assert torch.allclose(lse[sl], ref_lse[sl], rtol=1e-6, atol=1e-5), b
            assert torch.allclose(lp[sl], ref_lp[sl], rtol=1e-5, atol=1e-5), b


@pytest.mark.parametrize("impl", IMPLS)
def test_strided_hidden_and_target_errors(device, impl):
    """A hidden view with a padded row stride; out-of-range targets raise as
    torch.gather does; the tile path refuses float32 and hidden sizes that
    are not multiples of 128 (the chunked path takes them:
    test_gpu_linear_chunked)."""

    B, T, H, V = 2, 40, 256, 1000
    h, w, x, t, _old, _adv, _mask = _inputs(45, B, T, H, V)
    big = torch.zeros(B, T, H + 64, dtype=torch.bfloat16)
    big[..., :H] = h
    hv = big.to(device)[..., :H]
    with _tap(impl) as rec:
        lp = R.linear_token_logprobs(hv, w.to(device), t.to(device), impl=impl)
    _logp_check_impl(impl, lp, x, t, rec, h, w)
    bad = t.clone()
    bad[1, 3] = V
    with pytest.raises(RuntimeError, match="out of bounds"):
        R.linear_token_logprobs(h.to(device), w.to(device), bad.to(device), impl=impl)
    bad[1, 3] = -1
    with pytest.raises(RuntimeError, match="out of bounds"):
        R.linear_token_logprobs(h.to(device), w.to(device), bad.to(device), impl=impl)
    if impl == "tiles":
        with pytest.raises(TypeError, match="bfloat16"):
            R.linear_token_logprobs(h.float().to(device), w.float().to(device), t.to(device),
                                    impl=impl)
        with pytest.raises(ValueError, match="multiple of 128"):
            R.linear_token_logprobs(h[..., :200].to(device), w[:, :200].to(device), t.to(device),
                                    impl=impl)


@pytest.mark.parametrize("impl", IMPLS)
def test_fused_linear_grad_scale_and_diagnostic_grads(device, impl):
    """3 * loss scales both gradients; a loss that also differentiates a
    diagnostic (the KL term) equals the composition
    linear_token_logprobs -> clipped_policy_loss."""

    B, T, H, V = 8, 48, 128, 4104
    h, w, x, t, old, adv, mask = _inputs(46, B, T, H, V)
    d = lambda z: z.to(device)  # noqa: E731

    def run(fused, f):
        hd = d(h).requires_grad_()
        wd = d(w).requires_grad_()
        if fused:
            out = R.fused_linear_policy_loss(hd, wd, d(t), d(old), d(adv), d(mask), impl=impl,
                                             **KW["clipped"])
        else:
            lp = R.linear_token_logprobs(hd, wd, d(t), impl=impl)
            out = R.clipped_policy_loss(lp, d(old), d(adv), d(mask), **KW["clipped"])
        f(out).backward()
        return out, hd.grad, wd.grad

    o1, h1, w1 = run(True, lambda out: out.loss)
    o3, h3, w3 = run(True, lambda out: 3.0 * out.loss)
    # d hidden: each side rounded to bf16 once, within two bf16 ulps (the
    # chunked path: row-norm-wise, its GEMM's reduction order may vary from
    # run to run); d weight sums per-token terms that the dW pass rounds to
    # bf16 (3 g (onehot - p) against g (onehot - p)), so its rows agree
    # norm-wise
    if impl == "tiles":
        torch.testing.assert_close(h3.float(), 3.0 * h1.float(), rtol=2.0 ** -6, atol=1e-6)
    else:
        # the stored bf16 rows scaled by 3 (one more rounding) against another
        # run's rows times 3
        _same_grads(h3, 3.0 * h1.float(), impl, "3 x d hidden", tol=2.0 ** -6)
    num = (w3.float() - 3.0 * w1.float()).norm(dim=-1)
    den = (3.0 * w1.float()).norm(dim=-1)
    assert bool((num <= 1e-2 * den + 1e-12).all()), float((num / den.clamp_min(1e-30)).max())
    _ok, hk, wk = run(True, lambda out: out.loss + 0.5 * out.approximate_kl)
    _oc, hc, wc = run(False, lambda out: out.loss + 0.5 * out.approximate_kl)
    if impl == "tiles":
        assert torch.equal(hk, hc) and torch.equal(wk, wc)
    else:
        # the fused sweep's log-probs (the single-pass row kernel) and the
        # composition's (the log-prob row kernel) agree to float32 rounding,
        # and so do the d loss / d logp built on them
        torch.testing.assert_close(hk.float(), hc.float(), rtol=2.0 ** -7, atol=1e-6)
        torch.testing.assert_close(wk.float(), wc.float(), rtol=2.0 ** -7, atol=1e-6)


@pytest.mark.parametrize("impl", IMPLS)
def test_fused_linear_equals_logits_level_path(device, impl):
    """The loss of the LM-head path equals fused_policy_loss on the logits it
    consumes (float32 products for the tile path, the GEMM's bf16 products
    for the chunked path) within the log-probs' float32 accumulation error."""

    B, T, H, V = 8, 64, 256, 8256
    h, w, x, t, old, adv, mask = _inputs(47, B, T, H, V)
    d = lambda z: z.to(device)  # noqa: E731
    out_l, lp_l = R.fused_linear_policy_loss(d(h), d(w).requires_grad_(), d(t), d(old), d(adv),
                                             d(mask), return_logprobs=True, impl=impl,
                                             **KW["clipped"])
    if impl == "tiles":
        xd = d(x.float()).requires_grad_()
    else:
        xd = torch.mm(d(h).reshape(-1, H), d(w).t()).reshape(B, T, V).requires_grad_()
    out_x, lp_x = R.fused_policy_loss(xd, d(t), d(old), d(adv), d(mask), return_logprobs=True,
                                      **KW["clipped"])
    assert float((lp_l - lp_x).abs().max()) < 1e-4
    torch.testing.assert_close(out_l.loss, out_x.loss, rtol=1e-4, atol=1e-7)
    assert math.isfinite(out_l.loss.item())
