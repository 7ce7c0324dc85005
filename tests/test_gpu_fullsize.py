"""The hot path at the benchmark configs' full sizes (configs 2, 3 and 4; config
1 compared with the oracle on every row; config 5's LM head, both
implementations, against float64 pins formed without the kernels under
test), checked through what does not depend on size:

* a random sample of token rows against the float64 oracle (log-probs, and
  dlogits rebuilt from the oracle's d loss / d logp over the whole batch);
* every row's dlogits sums to zero (softmax rows sum to one) within the
  16-bit output rounding;
* masked tokens' dlogits rows are exactly zero;
* the loss against the oracle objective evaluated in float64 on the returned
  log-probs;
* skip_masked_rows=True is bit-identical to the default (config 2).

Inputs come from bench.py's generator (same distributions and seeds).  Each
test frees its tensors; config 4 writes dlogits in place (159 GB of logits).
"""

from __future__ import annotations

import gc

import numpy as np
import pytest
import torch

import bench
from oracle import roserlhf_oracle as o
from rosellm_amd import roserlhf as R

pytestmark = pytest.mark.gpu

N_SAMPLE = 48


def _free():
    gc.collect()
    torch.cuda.empty_cache()


def _sample_rows(N, mask, seed):
    """Half masked-in rows, a quarter masked-out rows, the rest uniform."""

    g = torch.Generator().manual_seed(seed)
    m = mask.reshape(-1).cpu()
    on = torch.nonzero(m).reshape(-1)
    off = torch.nonzero(~m).reshape(-1)
    pick = [on[torch.randint(0, on.numel(), (N_SAMPLE // 2,), generator=g)],
            torch.randint(0, N, (N_SAMPLE // 4,), generator=g)]
    if off.numel():
        pick.append(off[torch.randint(0, off.numel(), (N_SAMPLE // 4,), generator=g)])
    return torch.unique(torch.cat(pick))


def _check_rows(x_rows, t_rows, lp_rows, dl_rows, g_rows, what):
    """Sampled rows against the float64 oracle."""

    lpo = o.token_logprobs(x_rows, t_rows, exact=True)
    err = (lp_rows.double() - lpo).abs()
    bound = 1e-5 * lpo.abs() + 1e-7
    assert bool((err <= bound).all()), f"{what}: logp worst {float((err / bound).max()):.2f}x tol"
    p = torch.softmax(x_rows.double(), dim=-1)
    oh = torch.zeros_like(p)
    oh.scatter_(1, t_rows.long()[:, None], 1.0)
    want = g_rows.double()[:, None] * (oh - p)
    rounded = want.float().to(dl_rows.dtype).double()
    got = dl_rows.double()
    num = (got - rounded).norm(dim=-1)
    den = rounded.norm(dim=-1)
    rel = torch.where(den > 0, num / den.clamp_min(1e-300), num)
    assert float(rel.max()) <= 2e-3, f"{what}: dlogits row-norm err {float(rel.max()):.3e}"


def _row_sums_vanish(dl, what, chunk=8192):
    """sum_v dlogits[r, v] = g (1 - sum_v p_v) = 0 up to the output rounding."""

    flat = dl.reshape(-1, dl.shape[-1])
    worst = 0.0
    for r0 in range(0, flat.shape[0], chunk):
        c = flat[r0:r0 + chunk].float()
        s = c.sum(dim=-1).abs()
        a = c.abs().sum(dim=-1)
        worst = max(worst, float(torch.where(a > 0, s / a.clamp_min(1e-30), s).max()))
        del c
    assert worst <= 2.0 ** -7, f"{what}: |row sum| / sum|row| = {worst:.3e}"


def _masked_rows_zero(dl, mask, what, chunk=8192):
    flat = dl.reshape(-1, dl.shape[-1])
    m = mask.reshape(-1)
    for r0 in range(0, flat.shape[0], chunk):
        rows = ~m[r0:r0 + chunk]
        assert int(torch.count_nonzero(flat[r0:r0 + chunk][rows])) == 0, what


def _oracle_g(kind, lp, old, adv, mask, **kw):
    """d loss / d logp of the oracle objective in float64 over the whole batch,
    evaluated on the GPU's log-probs (pinned above on the sampled rows)."""

    cur = lp.detach().double().cpu().requires_grad_()
    fn = {"ppo": o.ppo_clip, "sapo": o.sapo, "gspo": o.gspo, "gspo_token": o.gspo_token}[kind]
    out = fn(cur, old.double().cpu(), adv.double().cpu(), mask.cpu(), **kw)
    out["loss"].backward()
    return out, cur.grad.reshape(-1)


def test_config1_fullsize_every_row(device):
    """Config 1 in full (32 x 128 rows of 50257 float32 logits, rows 4-byte
    aligned: the register-resident kernel's head/tail variant) against the
    float64 oracle on every row, for the fused path and for the composed
    path (gather_token_logprobs, clipped_policy_loss, autograd)."""

    print("[fullsize] config 1 every row", flush=True)
    cfg = bench.CONFIGS["c1"]
    with torch.no_grad():
        inp = bench.make_inputs(cfg, device, 1234)
    B, T, V = inp["B"], inp["T"], inp["V"]
    x, t, old, mask = inp["logits"], inp["actions"], inp["old"], inp["mask"]
    adv = R.group_standardized_advantages(inp["rewards"]).reshape(-1)[:, None].expand(B, T)
    kw = cfg["kw"]
    xc, tc, oc, ac, mc = (v.detach().cpu() for v in (x, t, old, adv, mask))
    out_o, lpo, dlo = o.policy_step("ppo", xc, tc, oc, ac.contiguous(), mc, exact=True, **kw)
    g = out_o["dloss_dlogp"]
    scale = max(abs(float(out_o["loss"])), float(ac.abs().mean()))
    for path in ("fused", "composed"):
        xd = x.detach().clone().requires_grad_()
        if path == "fused":
            out, lp = R.fused_policy_loss(xd, t, old, adv, mask, return_logprobs=True, **kw)
        else:
            lp = R.gather_token_logprobs(xd, t)
            out = R.clipped_policy_loss(lp, old, adv, mask, **kw)
        out.loss.backward()
        err = (lp.detach().double().cpu() - lpo).abs()
        assert bool((err <= 1e-5 * lpo.abs() + 1e-7).all()), (path, float(err.max()))
        assert abs(float(out.loss) - float(out_o["loss"])) <= 1e-5 * scale, path
        e = (xd.grad.double().cpu() - dlo).abs().reshape(-1, V).max(dim=-1).values
        bound = 1e-5 * g.reshape(-1).abs() + 1e-12
        assert bool((e <= bound).all()), (path, float((e / bound).max()))
        del xd
    del x, inp
    _free()


def test_config2_grpo_fullsize(device):
    print("[fullsize] config 2 fused GRPO", flush=True)
    cfg = bench.CONFIGS["c2"]
    with torch.no_grad():
        inp = bench.make_inputs(cfg, device, 1234)
    B, T, V = inp["B"], inp["T"], inp["V"]
    x, t, old, mask = inp["logits"], inp["actions"], inp["old"], inp["mask"]
    adv = R.group_standardized_advantages(inp["rewards"]).reshape(-1)[:, None].expand(B, T)
    kw = cfg["kw"]
    xd = x.requires_grad_()
    out, lp = R.fused_policy_loss(xd, t, old, adv, mask, return_logprobs=True, **kw)
    out.loss.backward()
    dl = xd.grad
    assert dl.dtype == torch.bfloat16 and dl.shape == x.shape
    out_o, g = _oracle_g("ppo", lp, old, adv, mask, **kw)
    scale = max(abs(float(out_o["loss"])), float(adv.abs().mean()))
    assert abs(float(out.loss) - float(out_o["loss"])) <= 1e-5 * scale
    for f in ("approximate_kl", "clip_fraction", "mean_ratio"):
        assert abs(float(getattr(out, f)) - float(out_o[f])) <= 1e-5 * max(1.0, abs(float(out_o[f])))
    rows = _sample_rows(B * T, mask, 7)
    xf = x.detach().reshape(-1, V)
    _check_rows(xf[rows.to(device)].cpu(), t.reshape(-1)[rows.to(device)].cpu(),
                lp.reshape(-1)[rows.to(device)].cpu(), dl.reshape(-1, V)[rows.to(device)].cpu(),
                g[rows], "c2")
    _row_sums_vanish(dl, "c2")
    _masked_rows_zero(dl, mask, "c2")
    # skip_masked_rows: same loss and dlogits, bit for bit
    loss0 = out.loss.detach().clone()
    xd.grad = None
    out2 = R.fused_policy_loss(xd, t, old, adv, mask, skip_masked_rows=True, **kw)
    out2.loss.backward()
    assert torch.equal(out2.loss, loss0)
    flat0, flat1 = dl.reshape(-1, V), xd.grad.reshape(-1, V)
    for r0 in range(0, B * T, 16384):
        assert torch.equal(flat0[r0:r0 + 16384], flat1[r0:r0 + 16384]), r0
    del xd, x, dl, flat0, flat1, out, out2, inp
    _free()


@pytest.mark.parametrize("objective", ["gspo", "gspo_token"])
def test_config3_gspo_fullsize(device, objective):
    print(f"[fullsize] config 3 {objective}", flush=True)
    cfg = bench.CONFIGS["c3"]
    with torch.no_grad():
        inp = bench.make_inputs(cfg, device, 1234)
    B, T, V = inp["B"], inp["T"], inp["V"]
    x, t, old, mask = inp["logits"], inp["actions"], inp["old"], inp["mask"]
    seq = R.group_standardized_advantages(inp["rewards"]).reshape(-1)
    adv = seq if objective == "gspo" else seq[:, None].expand(B, T)
    kw = cfg["kw"]
    xd = x.requires_grad_()
    out, lp = R.fused_policy_loss(xd, t, old, adv, mask, objective=objective,
                                  return_logprobs=True, **kw)
    out.loss.backward()
    dl = xd.grad
    out_o, g = _oracle_g(objective, lp, old, adv, mask, **kw)
    scale = max(abs(float(out_o["loss"])), float(seq.abs().mean()))
    assert abs(float(out.loss) - float(out_o["loss"])) <= 1e-5 * scale
    torch.testing.assert_close(out.sequence_ratios.double().cpu(), out_o["sequence_ratios"],
                               rtol=1e-5, atol=1e-7)
    rows = _sample_rows(B * T, mask, 8)
    xf = x.detach().reshape(-1, V)
    r_d = rows.to(device)
    _check_rows(xf[r_d].cpu(), t.reshape(-1)[r_d].cpu(), lp.reshape(-1)[r_d].cpu(),
                dl.reshape(-1, V)[r_d].cpu(), g[rows], f"c3 {objective}")
    _row_sums_vanish(dl, f"c3 {objective}")
    _masked_rows_zero(dl, mask, f"c3 {objective}")
    del xd, x, dl, out, inp
    _free()


def test_config4_gae_sapo_inplace_fullsize(device):
    print("[fullsize] config 4 GAE + whitening + SAPO, in place", flush=True)
    cfg = bench.CONFIGS["c4"]
    with torch.no_grad():
        inp = bench.make_inputs(cfg, device, 1234)
    B, T, V = inp["B"], inp["T"], inp["V"]
    x, t, old, mask = inp["logits"], inp["actions"], inp["old"], inp["mask"]
    rows = _sample_rows(B * T, mask, 9)
    r_d = rows.to(device)
    x_rows = x.reshape(-1, V)[r_d].cpu()  # kept before the logits are overwritten
    # estimators against the oracle's sequential recurrences
    adv, ret = R.generalized_advantage_estimation(inp["rewards"], inp["values"], gamma=1.0,
                                                  gae_lambda=0.95, valid_mask=mask)
    adv_o, ret_o = o.gae(inp["rewards"].double().cpu(), inp["values"].double().cpu(), gamma=1.0,
                         gae_lambda=0.95, valid_mask=mask.cpu())
    tol = 1e-5 * max(1.0, float(adv_o.abs().max()))
    assert float((adv.double().cpu() - adv_o).abs().max()) <= tol
    assert float((ret.double().cpu() - ret_o).abs().max()) <= tol
    assert bool((adv.cpu()[~mask.cpu()] == 0).all())
    w = R.masked_whiten(adv, mask)
    sel = w.double()[mask]
    assert abs(float(sel.mean())) < 1e-5 and abs(float(sel.std(unbiased=False)) - 1) < 1e-5
    kw = cfg["kw"]
    xd = x.requires_grad_()
    out, lp = R.fused_policy_loss(xd, t, old, w, mask, objective="sapo", inplace=True,
                                  return_logprobs=True, **kw)
    out.loss.backward()
    dl = xd.grad
    assert dl.data_ptr() == x.data_ptr()  # written in place
    out_o, g = _oracle_g("sapo", lp, old, w, mask, **kw)
    scale = max(abs(float(out_o["loss"])), float(w.abs().mean()))
    assert abs(float(out.loss) - float(out_o["loss"])) <= 1e-5 * scale
    _check_rows(x_rows, t.reshape(-1)[r_d].cpu(), lp.reshape(-1)[r_d].cpu(),
                dl.reshape(-1, V)[r_d].cpu(), g[rows], "c4")
    _row_sums_vanish(dl, "c4")
    _masked_rows_zero(dl, mask, "c4")
    del xd, x, dl, out, inp
    _free()


def _rows_close(a, b, tol, what, chunk=16384):
    """Row-wise ||a - b|| <= tol * ||b|| (rows of the last dimension)."""

    fa, fb = a.reshape(-1, a.shape[-1]), b.reshape(-1, b.shape[-1])
    worst = 0.0
    for r0 in range(0, fa.shape[0], chunk):
        x, y = fa[r0:r0 + chunk].float(), fb[r0:r0 + chunk].float()
        num, den = (x - y).norm(dim=-1), y.norm(dim=-1)
        worst = max(worst, float(torch.where(den > 0, num / den.clamp_min(1e-30), num).max()))
    assert worst <= tol, f"{what}: worst row-norm rel diff {worst:.3e}"
    return worst


@pytest.mark.parametrize("impl,objective", [("chunked", "clipped"), ("tiles", "clipped"),
                                            ("chunked", "gspo")])
def test_config5_linear_fullsize_against_exact_rows(device, impl, objective):
    """Config 5 in full (262144 tokens, hidden 1024, V = 151936 bf16) through
    both LM-head implementations, pinned without the kernels under test:

    * every token's log-sum-exp and target logit come from float64 products
      of the bf16 hidden states and weight, formed on the GPU with torch in
      float64, 2048 tokens at a time (for the chunked path rounded to bf16
      first, through float32 as its GEMM's float32 accumulator rounds them:
      the logits it consumes);
    * d loss / d logp comes from oracle.ppo_clip (GSPO: oracle.gspo, config
      3's clip band, per-sequence advantages) in float64 on the CPU, over all
      262144 tokens, on those log-probs.  GSPO takes the chunked path's other
      backward: every log-prob first, then the active blocks' logits formed
      a second time.

    Checks: every token's log-prob (the bars of test_gpu_linear for each
    implementation); the d hidden rows of 64 random tokens and the d weight
    rows of 8 random vocabulary entries (each a sum over all 262144 tokens)
    within twice the propagated one-ulp bound of the bf16 dlogits."""

    from test_gpu_linear import _ulp16

    print(f"[fullsize] config 5 LM head ({impl}, {objective}) vs float64 pins", flush=True)
    cfg = bench.CONFIGS["c5"]
    with torch.no_grad():
        inp = bench.make_inputs(cfg, device, 1234)
    B, T = inp["B"], inp["T"]
    h, w = inp["hidden"], inp["weight"]
    t, old, mask = inp["actions"], inp["old"], inp["mask"]
    adv_seq = R.group_standardized_advantages(inp["rewards"]).reshape(-1)
    adv = adv_seq[:, None].expand(B, T)
    kw = cfg["kw"] if objective == "clipped" else bench.CONFIGS["c3"]["kw"]
    adv_arg = adv if objective == "clipped" else adv_seq
    del inp
    _free()
    N, H, V = B * T, h.shape[-1], w.shape[0]
    hd, wd = h.detach().clone().requires_grad_(), w.detach().clone().requires_grad_()
    out, lp = R.fused_linear_policy_loss(hd, wd, t, old, adv_arg, mask, return_logprobs=True,
                                         impl=impl, objective=objective, **kw)
    out.loss.backward()
    gh, gw = hd.grad, wd.grad
    del hd, wd, out
    _free()
    gen = torch.Generator().manual_seed(77)
    idx = torch.randperm(N, generator=gen)[:64]
    vs = torch.randperm(V, generator=gen)[:8]
    idx_d, vs_d = idx.to(device), vs.to(device)
    t_flat = t.reshape(-1)
    with torch.no_grad():
        h64 = h.reshape(N, H).double()
        w64 = w.double()
        lse64 = torch.empty(N, dtype=torch.float64, device=device)
        xt64 = torch.empty(N, dtype=torch.float64, device=device)
        xmax = torch.empty(N, dtype=torch.float64, device=device)
        xv64 = torch.empty(N, 8, dtype=torch.float64, device=device)
        rows64 = torch.empty(64, V, dtype=torch.float64, device=device)
        for r0 in range(0, N, 2048):
            r1 = min(N, r0 + 2048)
            x = h64[r0:r1] @ w64.t()
            if impl == "chunked":
                x = x.float().to(torch.bfloat16).double()
            lse64[r0:r1] = torch.logsumexp(x, dim=-1)
            xt64[r0:r1] = x.gather(1, t_flat[r0:r1, None]).squeeze(1)
            xmax[r0:r1] = x.abs().amax(dim=-1)
            xv64[r0:r1] = x[:, vs_d]
            sel = torch.nonzero((idx_d >= r0) & (idx_d < r1)).reshape(-1)
            if sel.numel():
                rows64[sel] = x[idx_d[sel] - r0]
            del x
        lp_ref = xt64 - lse64
        # 1. every token's log-prob
        err = (lp.reshape(-1).double() - lp_ref).abs()
        bound = 1e-5 * lp_ref.abs() + 1e-6
        if impl == "chunked":
            bound = bound + _ulp16(xt64.abs().cpu()).to(device) + _ulp16(xmax.cpu()).to(device)
        worst = float((err / bound).max())
        print(f"[fullsize] c5 {impl} {objective}: every log-prob, max err/bound {worst:.3f} "
              f"(max abs err {float(err.max()):.2e})", flush=True)
        assert worst <= 1.0
    # d loss / d logp from the float64 oracle on the CPU
    cur = lp_ref.cpu().view(B, T).requires_grad_()
    if objective == "clipped":
        res = o.ppo_clip(cur, old.double().cpu(), adv.double().cpu(), mask.cpu(), **kw)
    else:
        res = o.gspo(cur, old.double().cpu(), adv_seq.double().cpu(), mask.cpu(), **kw)
    res["loss"].backward()
    g = cur.grad.reshape(-1).to(device)
    with torch.no_grad():
        # 2. d hidden rows of 64 tokens
        p = torch.exp(rows64 - lse64[idx_d, None])
        oh = torch.zeros_like(p).scatter_(1, t_flat[idx_d][:, None], 1.0)
        dl16 = (g[idx_d][:, None] * (oh - p)).to(torch.bfloat16).double()
        ref = dl16 @ w64
        prop = _ulp16(dl16.cpu()).to(device) @ w64.abs()
        got = gh.reshape(N, H)[idx_d].double()
        den = 2 * prop + _ulp16((ref.abs() + prop).cpu()).to(device) + 1e-30
        excess = float(((got - ref).abs() / den).max())
        print(f"[fullsize] c5 {impl} {objective}: d hidden rows max |err|/bound {excess:.3f}",
              flush=True)
        assert excess <= 1.0
        # 3. d weight rows of 8 vocabulary entries, summed over every token
        pv = torch.exp(xv64 - lse64[:, None])
        ohv = (t_flat[:, None] == vs_d[None, :]).double()
        dlv = (g[:, None] * (ohv - pv)).to(torch.bfloat16).double()
        refw = dlv.t() @ h64
        propw = _ulp16(dlv.cpu()).to(device).t() @ h64.abs()
        gotw = gw[vs_d].double()
        denw = 2 * propw + _ulp16((refw.abs() + propw).cpu()).to(device) + 1e-30
        excess_w = float(((gotw - refw).abs() / denw).max())
        print(f"[fullsize] c5 {impl} {objective}: d weight rows max |err|/bound {excess_w:.3f}",
              flush=True)
        assert excess_w <= 1.0
    del gh, gw, h, w, lp, h64, w64, lse64, xt64, xmax, xv64, rows64, g
    _free()
