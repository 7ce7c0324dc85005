"""SFT next-token cross-entropy (rosetrainer/model.py:643-649) on the HIP row
kernels vs the CPU oracle, on identical seeded inputs (MI355X).

Bars as for the policy losses: float32 losses within 1e-5 relative; 16-bit
logits: loss within 2e-3 relative (the float32 arithmetic lands far inside
it), dlogits rows within 2e-3 norm-wise of the correctly rounded exact rows
and every element within one ulp of it; float32 dlogits within 1e-5 of |g|
per row.  Exact expectations are the float64 evaluation of the same math.
The LM-head form is held to the propagated bound of test_gpu_linear.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import roserlhf_oracle as o
from rosellm_amd import rosetrainer as RT

from test_gpu_linear import _consumed, _product_check, _tap
from test_gpu_parity import _close_rows_by_g, _rownorm16, _ulp16

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _labels(g, shape, V, frac_ignored=0.2, ignore=-100):
    y = torch.randint(0, V, shape, generator=g)
    y[torch.rand(shape, generator=g) < frac_ignored] = ignore
    return y


def _dominant(x, g, frac=0.05, bump=15.0):
    """Give a fraction of rows one dominant logit (+bump), as config 2."""

    V = x.shape[-1]
    rows = x.reshape(-1, V)
    pick = torch.rand(rows.shape[0], generator=g) < frac
    col = torch.randint(0, V, (rows.shape[0],), generator=g)
    rows[pick, col[pick]] += bump
    return x


@pytest.mark.parametrize("reduction", ["mean", "sum"])
def test_cross_entropy_f32_unaligned_rows(device, reduction):
    """float32 [N, V] with V = 50257: rows not 16-byte aligned, the
    register-resident kernel's head/tail variant."""

    print(f"[sft-f32] reduction={reduction}", flush=True)
    g = _gen(101)
    N, V = 300, 50257
    x = torch.randn(N, V, generator=g) * 2.0
    y = _labels(g, (N,), V)
    xd = x.to(device).requires_grad_()
    loss = RT.cross_entropy(xd, y.to(device), reduction=reduction)
    loss.backward()
    want, dl = o.sft_step(x, y, causal=False, reduction=reduction, exact=True)
    assert loss.dtype == torch.float32
    assert abs(loss.item() - want.item()) <= 1e-5 * abs(want.item())
    n = int((y != -100).sum())
    gabs = torch.where(y != -100, torch.full((N,), 1.0 if reduction == "sum" else 1.0 / n),
                       torch.zeros(N))
    _close_rows_by_g(xd.grad, dl, gabs, 1e-5, "dlogits f32")
    assert (xd.grad[y.to(device) == -100] == 0).all()


@pytest.mark.parametrize("dtype,V", [(torch.bfloat16, 32768), (torch.float16, 4096),
                                     (torch.bfloat16, 32001)])
def test_causal_lm_loss_16bit(device, dtype, V):
    """[B, T, V] causal shift through strided views; V % 8 == 0 takes the
    register-resident kernel's plain variant, V = 32001 its head/tail variant."""

    print(f"[sft-causal] dtype={dtype} V={V}", flush=True)
    g = _gen(102)
    B, T = 4, 65
    x = _dominant(torch.randn(B, T, V, generator=g) * 3.0, g).to(dtype)
    y = _labels(g, (B, T), V)
    xd = x.to(device).requires_grad_()
    loss = RT.causal_lm_loss(xd, y.to(device))
    loss.backward()
    want, dl = o.sft_step(x, y, causal=True, exact=True)
    assert loss.dtype == torch.float32
    rel = abs(loss.item() - want.item()) / abs(want.item())
    print(f"loss rel err {rel:.3e}", flush=True)
    assert rel <= 2e-3
    assert rel <= 1e-5  # float32 arithmetic on exact upcasts
    assert xd.grad.dtype == dtype and xd.grad.shape == x.shape
    assert (xd.grad[:, -1] == 0).all()
    _rownorm16(xd.grad, dl, 2e-3, "dlogits 16-bit")
    same = _ulp16(xd.grad, dl, "dlogits 16-bit")
    assert same >= 0.98, same


def test_causal_lm_loss_matches_reference_expression_and_custom_ignore(device):
    """ignore_index = 0 (token 0 carries no loss) and reduction "sum"; the
    oracle is the reference's own expression shape (shift, view, F.cross_entropy)."""

    g = _gen(103)
    B, T, V = 3, 40, 8192
    x = (torch.randn(B, T, V, generator=g) * 3.0).to(torch.bfloat16)
    y = torch.randint(0, 6, (B, T), generator=g)  # many zeros
    xd = x.to(device).requires_grad_()
    loss = RT.causal_lm_loss(xd, y.to(device), ignore_index=0, reduction="sum")
    loss.backward()
    want, dl = o.sft_step(x, y, causal=True, ignore_index=0, reduction="sum", exact=True)
    assert abs(loss.item() - want.item()) <= 1e-5 * abs(want.item())
    _rownorm16(xd.grad, dl, 2e-3, "dlogits ignore=0 sum")
    # -100 is now an ordinary (out of range) id
    y2 = y.clone()
    y2[1, 7] = -100
    with pytest.raises(IndexError, match="out of bounds"):
        RT.causal_lm_loss(x.to(device), y2.to(device), ignore_index=0)


def test_all_ignored_and_range_errors(device):
    g = _gen(104)
    x = (torch.randn(2, 9, 4096, generator=g)).to(torch.bfloat16)
    xd = x.to(device).requires_grad_()
    loss = RT.causal_lm_loss(xd, torch.full((2, 9), -100, device=device))
    assert math.isnan(loss.item())
    loss.backward()
    assert (xd.grad == 0).all()
    y = torch.randint(0, 4096, (2, 9), generator=g)
    y[0, 3] = 4096
    with pytest.raises(IndexError, match="out of bounds"):
        RT.causal_lm_loss(x.to(device), y.to(device))
    y[0, 3] = -5
    with pytest.raises(IndexError, match="out of bounds"):
        RT.cross_entropy(x.to(device).reshape(-1, 4096), y.reshape(-1).to(device))
    # int32 labels are accepted as well
    y[0, 3] = 11
    l64 = RT.causal_lm_loss(x.to(device), y.to(device))
    l32 = RT.causal_lm_loss(x.to(device), y.to(device, torch.int32))
    assert torch.equal(l64, l32)


def test_inplace_and_upstream_scale(device):
    g = _gen(105)
    B, T, V = 2, 50, 16384
    x = (torch.randn(B, T, V, generator=g) * 3.0).to(torch.bfloat16)
    y = _labels(g, (B, T), V)
    a = x.to(device).requires_grad_()
    RT.causal_lm_loss(a, y.to(device)).backward()
    b = x.to(device).requires_grad_()
    (2.5 * RT.causal_lm_loss(b, y.to(device))).backward()
    torch.testing.assert_close(b.grad.float(), 2.5 * a.grad.float(), rtol=8e-3, atol=1e-9)
    # inplace: the gradient is written over the logits, bit-identical
    buf = x.to(device).detach()
    loss_c = RT.causal_lm_loss(buf.requires_grad_(), y.to(device), inplace=True)
    loss_a = RT.causal_lm_loss(x.to(device), y.to(device))
    assert torch.equal(loss_c, loss_a)
    assert torch.equal(buf.detach(), a.grad), "in-place gradient differs"


@pytest.mark.parametrize("layout", ["padded_vocab", "shifted_rows"])
def test_inplace_strided_views_upstream_scale(device, layout):
    """In place on a strided view, with an upstream gradient of 2.5: every
    gradient row of the view is the unscaled in-place gradient (same view,
    same kernel) times 2.5, rounded once to bf16; the unscaled gradient
    matches the out-of-place one; memory outside the view is untouched."""

    print(f"[sft-inplace-strided] layout={layout}", flush=True)
    g = _gen(107)
    B, T, V, PAD = 3, 40, 4104, 56
    full = (torch.randn(B, T, V + PAD, generator=g) * 3.0).to(torch.bfloat16)
    y = _labels(g, (B, T), V)

    def view_of(buf):
        return buf[..., :V] if layout == "padded_vocab" else buf[:, :-1, :V]

    lab = (y if layout == "padded_vocab" else y[:, 1:]).to(device)
    grads = []
    for upstream in (1.0, 2.5):
        buf = full.to(device)
        leaf = view_of(buf).detach().requires_grad_()
        (upstream * RT.cross_entropy(leaf, lab, inplace=True)).backward()
        torch.cuda.synchronize()
        grads.append(leaf.detach().clone())
        host = buf.cpu()
        assert torch.equal(host[..., V:], full[..., V:]), "padding columns were written"
        if layout == "shifted_rows":
            assert torch.equal(host[:, -1], full[:, -1]), "rows outside the view were written"
    g1, g25 = grads
    assert torch.equal(g25, (g1.float() * 2.5).to(torch.bfloat16)), "rows scaled wrongly"
    a = view_of(full).contiguous().to(device).requires_grad_()
    RT.cross_entropy(a, lab).backward()
    # another kernel variant (rows off 128-byte boundaries): within one bf16 ulp
    same = _ulp16(g1, a.grad.float(), "in place vs out of place")
    assert same >= 0.98, same


@pytest.mark.parametrize("impl", ["tiles", "chunked"])
@pytest.mark.parametrize("ignore_index", [-100, 0])
def test_linear_causal_lm_loss(device, ignore_index, impl):
    """LM head + shift + cross-entropy without the whole logits tensor: loss
    vs the float64 chain on the logits the implementation consumed (the exact
    products for the tile path; the chunked path's bf16 GEMM outputs, recorded
    and pinned to the exact products); dhidden and dW within the propagated
    bound of the bf16 dlogits; ignored labels carry nothing."""

    print(f"[sft-linear] impl={impl} ignore_index={ignore_index}", flush=True)
    g = _gen(106)
    B, T, H, V = 4, 97, 256, 8256
    h = torch.randn(B, T, H, generator=g).to(torch.bfloat16)
    w = (torch.randn(V, H, generator=g) * (2.0 / H ** 0.5)).to(torch.bfloat16)
    y = _labels(g, (B, T), V, ignore=ignore_index)
    hd = h.to(device).requires_grad_()
    wd = w.to(device).requires_grad_()
    with _tap(impl) as rec:
        loss = RT.linear_causal_lm_loss(hd, wd, y.to(device), ignore_index=ignore_index,
                                        impl=impl)
        loss.backward()
    hs = h[:, :-1].contiguous()
    x, xb = _consumed(impl, rec, hs.double() @ w.double().t(), hs, w)
    want, dl = o.sft_step(x, y[:, 1:], causal=False, ignore_index=ignore_index, exact=True)
    assert abs(loss.item() - want.item()) <= 1e-5 * abs(want.item())
    if xb is not x:  # the backward's own recomputed logits
        _want_b, dl = o.sft_step(xb, y[:, 1:], causal=False, ignore_index=ignore_index,
                                 exact=True)
    dl = dl.double().reshape(-1, V)
    assert (hd.grad[:, -1] == 0).all()
    _product_check(hd.grad[:, :-1].reshape(-1, H), dl, w, "dhidden", transpose=False)
    _product_check(wd.grad, dl, hs.reshape(-1, H), "dweight", transpose=True)


@pytest.mark.parametrize("impl", ["tiles", "chunked"])
def test_ignored_labels_take_no_gradient_from_upstream(device, impl):
    """An ignored label's log-prob is the constant 0: a non-zero upstream
    gradient there must reach neither d hidden nor d weight.  The same
    backward with the upstream gradient zeroed on ignored labels is the
    expectation (bit-identical d hidden; d weight within one bf16 ulp, as the
    tile path's dW pass may visit, and split, different token tiles)."""

    from rosellm_amd.roserlhf import linear as LIN

    print(f"[sft-linear-ignored-g] impl={impl}", flush=True)
    g = _gen(107)
    B, T, H, V = 3, 130, 256, 4160
    h = torch.randn(B, T, H, generator=g).to(torch.bfloat16)
    w = (torch.randn(V, H, generator=g) * (2.0 / H ** 0.5)).to(torch.bfloat16)
    y = _labels(g, (B, T), V, frac_ignored=0.3)
    r = torch.randn(B, T, generator=g) + 2.0  # non-zero everywhere
    keep = (y != -100).float()

    def grads(up):
        hd = h.to(device).requires_grad_()
        wd = w.to(device).requires_grad_()
        lp = LIN.linear_label_logprobs(hd, wd, y.to(device), -100, impl=impl)
        (lp * up.to(device)).sum().backward()
        return lp.detach().cpu(), hd.grad.cpu(), wd.grad.cpu()

    lp_a, dh_a, dw_a = grads(r)
    lp_b, dh_b, dw_b = grads(r * keep)
    ign = y == -100
    assert ign.any() and (lp_a[ign] == 0).all()
    assert torch.equal(lp_a, lp_b)
    assert (dh_a[ign] == 0).all(), "an ignored label passed gradient to d hidden"
    assert torch.equal(dh_a, dh_b)
    from test_gpu_linear import _ulp16 as _bf16_ulp

    diff = (dw_a.double() - dw_b.double()).abs()
    assert (diff <= _bf16_ulp(dw_b.double()).abs() + 1e-30).all(), float(diff.max())
