"""rrl_logprob_bwd through the C ABI against the float64 oracle (MI355X).

dlogits = g * (onehot(target) - softmax(x)) (losses.py:34-38 backward, the
composed path's second read of the logits).  16-byte aligned rows that are a
whole number of 16-byte vectors take the register-resident kernel; the same call with
accumulate = 1 into zeros takes the generic row kernel, so the two are also
held against each other.  Float32 rows, odd vocabularies and rows that do not
start on a 16-byte boundary take the resident variant that carries the
row's head and tail elements beside the aligned slabs.  Bars as in
test_gpu_parity: 16-bit dlogits within one ulp of the correctly rounded exact
value per element (at least 98% bit-identical) and 2e-3 row-norm error;
float32 dlogits within 1e-5 of |g| per row; zero-gradient rows exactly zero;
an in-place call bit-identical to the out-of-place one.
"""

from __future__ import annotations

import pytest
import torch

from rosellm_amd import _native as nat

from test_gpu_parity import F32_RTOL, _close_rows_by_g, _rownorm16, _ulp16

pytestmark = pytest.mark.gpu


def _exact(x, t, g):
    """float64 lse, log-prob and dlogits of [B, T, V] logits; a target
    outside [0, V) has no one-hot column."""

    xd = x.double()
    lse = torch.logsumexp(xd, dim=-1)
    V = x.shape[-1]
    ok = (t >= 0) & (t < V)
    ts = torch.where(ok, t, torch.zeros_like(t))
    xt = xd.gather(-1, ts.unsqueeze(-1)).squeeze(-1)
    logp = torch.where(ok, xt - lse, torch.full_like(lse, float("nan")))
    gd = g.double()
    dl = -gd.unsqueeze(-1) * torch.exp(xd - lse.unsqueeze(-1))
    onehot = torch.zeros_like(dl).scatter_(-1, ts.unsqueeze(-1), 1.0) * ok.unsqueeze(-1)
    # g * (1 - p_t) = -g * expm1(logp) at the target column
    tcol = -gd * torch.expm1(torch.where(ok, logp, torch.zeros_like(logp)))
    dl = torch.where(onehot > 0, tcol.unsqueeze(-1).expand_as(dl), dl)
    return lse, logp, dl


def _bwd(x, t, lse, logp, g, out=None, accumulate=0):
    """One rrl_logprob_bwd call on [B, T, V] logits (any row strides)."""

    B, T, V = x.shape
    dl = out if out is not None else torch.empty(B, T, V, dtype=x.dtype, device=x.device)
    tv, _keep = nat.rows_view(t, B, T)
    nat.call("rrl_logprob_bwd", x.data_ptr(), nat.dtype_code(x.dtype), B, T, V,
             x.stride(0), x.stride(1), tv, lse.data_ptr(), logp.data_ptr(), g.data_ptr(),
             dl.data_ptr(), nat.dtype_code(dl.dtype), dl.stride(0), dl.stride(1), accumulate,
             nat.stream_ptr(x.device))
    return dl


def _inputs(seed, B, T, V, dtype, zero_rows=True, bad_targets=False):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, T, V, generator=g) * 3.0).to(dtype)
    t = torch.randint(0, V, (B, T), generator=g)
    up = torch.randn(B, T, generator=g)
    if zero_rows:
        up[torch.rand(B, T, generator=g) < 0.3] = 0.0
    if bad_targets and B * T >= 3:
        t.view(-1)[1] = -1
        t.view(-1)[2] = V
    return x, t, up


def _check(dl, want, what, g=None):
    if dl.dtype == torch.float32:
        _close_rows_by_g(dl, want, g, F32_RTOL, what)
        return
    exact = _ulp16(dl, want, what)
    assert exact > 0.98, (what, exact)
    _rownorm16(dl, want, 2e-3, what)


@pytest.mark.parametrize(
    "dtype,V,B,T",
    [
        (torch.bfloat16, 151936, 3, 7),  # config-2 vocabulary: 19 slabs per lane
        (torch.bfloat16, 65536, 2, 3),
        (torch.bfloat16, 20000, 2, 5),  # partial last slab
        (torch.float16, 4096, 3, 4),
        (torch.bfloat16, 8, 2, 3),  # one vector per row
        (torch.bfloat16, 4096, 4, 300),  # 1200 rows: several rows per workgroup
        # head / tail variant: rows off 16-byte boundaries, V not a multiple of 8 (4)
        (torch.float32, 50257, 2, 6),  # config-1 vocabulary
        (torch.float32, 81923, 1, 3),  # 20 slabs of float32 vectors
        (torch.float32, 7, 2, 3),  # head and tail only
        (torch.bfloat16, 50257, 3, 5),
        (torch.float16, 4099, 3, 4),
        (torch.bfloat16, 3, 2, 2),
        (torch.float32, 3001, 5, 60),  # 300 rows: every head offset, several rows per workgroup
    ],
)
@pytest.mark.parametrize("tdtype", [torch.int64, torch.int32])
def test_bwd_matches_oracle_and_generic(device, dtype, V, B, T, tdtype):
    print(f"[bwd] dtype={dtype} V={V} B={B} T={T} targets={tdtype}", flush=True)
    x, t, up = _inputs(V + B * T, B, T, V, dtype, bad_targets=True)
    lse, logp, want = _exact(x, t, up)
    xd, td = x.to(device), t.to(tdtype).to(device)
    lse_d, logp_d, g_d = (v.float().to(device) for v in (lse, logp, up))
    dl = _bwd(xd, td, lse_d, logp_d, g_d)
    torch.cuda.synchronize()
    _check(dl, want, "dlogits", up)
    zero = (up == 0).to(device)
    assert torch.count_nonzero(dl[zero]).item() == 0
    # accumulate = 1 into zeros runs the generic row kernel
    ref = _bwd(xd, td, lse_d, logp_d, g_d, out=torch.zeros_like(xd), accumulate=1)
    torch.cuda.synchronize()
    if dtype == torch.float32:
        _close_rows_by_g(dl, ref, up, F32_RTOL, "resident vs generic")
    else:
        _ulp16(dl, ref.float(), "resident vs generic")


def test_bwd_inplace_and_strided(device):
    """In place over the logits (the linear path's use) is bit-identical to
    out of place; logits[:, :-1] of a [B, T+1, V] tensor is read as a view."""

    B, T, V = 2, 9, 151936
    x, t, up = _inputs(5, B, T + 1, V, torch.bfloat16)
    t, up = t[:, :-1].contiguous(), up[:, :-1].contiguous()
    xs = x[:, :-1]
    lse, logp, want = _exact(xs, t, up)
    xd = x.to(device)
    td = t.to(device)
    lse_d, logp_d, g_d = (v.float().to(device) for v in (lse, logp, up))
    dl = _bwd(xd[:, :-1], td, lse_d, logp_d, g_d)
    torch.cuda.synchronize()
    _check(dl, want, "strided")
    xi = xd[:, :-1].contiguous()
    _bwd(xi, td, lse_d, logp_d, g_d, out=xi)
    torch.cuda.synchronize()
    assert torch.equal(xi.view(torch.int16), dl.view(torch.int16))


def test_bwd_extreme_logits(device):
    """A log-sum-exp of 3e38 (the 16-bit maximum region), a half -inf row and
    an all -inf row but one entry: no rerun is needed, the exponent is formed
    from x - lse."""

    B, T, V = 2, 4, 4096
    x, t, up = _inputs(11, B, T, V, torch.bfloat16, zero_rows=False)
    xf = x.float()
    xf[0, 0, 7] = 3.0e38
    t[0, 0] = 7
    xf[0, 1, 9] = 3.0e38
    t[0, 1] = 11
    xf[0, 2, : V // 2] = -float("inf")
    t[0, 2] = V - 3
    xf[1, 0, :] = -float("inf")
    xf[1, 0, 5] = 0.0
    t[1, 0] = 5
    x = xf.to(torch.bfloat16)
    lse, logp, want = _exact(x, t, up)
    d = lambda v: v.to(device)  # noqa: E731
    dl = _bwd(d(x), d(t), d(lse.float()), d(logp.float()), d(up))
    torch.cuda.synchronize()
    _check(dl, want, "extreme")


def test_bwd_resident_vs_generic_config3_fullsize(device):
    """Config 3's full shape (256 x 1024 rows, V = 151936 bf16, bench.py's
    inputs) with GSPO's gradient pattern: 70% of the sequences and the masked
    tokens have g = 0.  The register-resident backward and the generic row
    kernel (accumulate = 1 into zeros) agree within one bf16 ulp on every
    element; zero-gradient rows are exactly zero."""

    import gc

    import bench

    print("[bwd] config 3 full size: resident vs generic", flush=True)
    # Two 79.7 GB tensors (logits, dlogits) and one 5 GB block of reference
    # rows: start from an empty caching allocator.
    gc.collect()
    torch.cuda.empty_cache()
    cfg = bench.CONFIGS["c3"]
    with torch.no_grad():
        inp = bench.make_inputs(cfg, device, 1234)
    B, T, V = inp["B"], inp["T"], inp["V"]
    x, t, mask = inp["logits"], inp["actions"], inp["mask"]
    del inp
    # Release the input generator's temporaries before anything small can be
    # carved out of their cached segment and pin it.
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    N = B * T
    lse = torch.empty(N, device=device)
    logp = torch.empty(N, device=device)
    tv, _keep = nat.rows_view(t, B, T)
    nat.call("rrl_logprob_fwd", x.data_ptr(), nat.dtype_code(x.dtype), B, T, V, x.stride(0),
             x.stride(1), tv, logp.data_ptr(), nat.F32, lse.data_ptr(), None,
             nat.stream_ptr(device))
    gen = torch.Generator(device=device).manual_seed(99)
    g = torch.randn(B, T, device=device, generator=gen) * 1e-5
    seq_zero = torch.rand(B, 1, device=device, generator=gen) < 0.7
    g = torch.where(seq_zero | ~mask, torch.zeros_like(g), g)
    dl = _bwd(x, t, lse, logp, g)
    torch.cuda.synchronize()
    zero_rows = (g == 0).reshape(-1)
    worst, exact, total = 0, 0, 0
    dlf, xf, tf = dl.view(N, V), x.view(N, V), t.reshape(-1)
    block, chunk = 16384, 2048
    ref = torch.empty(1, block, V, dtype=x.dtype, device=device)
    for r0 in range(0, N, block):
        n = min(block, N - r0)
        # the generic row kernel (accumulate = 1 into zeros) on this block
        rb = ref[:, :n]
        rb.zero_()
        _bwd(xf[r0:r0 + n][None], tf[r0:r0 + n][None], lse[r0:], logp[r0:], g.reshape(-1)[r0:],
             out=rb, accumulate=1)
        for c0 in range(0, n, chunk):
            a_ = dlf[r0 + c0:r0 + c0 + chunk]
            b_ = rb[0, c0:c0 + chunk]
            dist = (_ord(a_) - _ord(b_)).abs()
            tiny = (a_.float() - b_.float()).abs() < 1e-30
            dist = torch.where(tiny, torch.zeros_like(dist), dist)
            worst = max(worst, int(dist.max()))
            exact += int((dist == 0).sum())
            total += dist.numel()
            zr = zero_rows[r0 + c0:r0 + c0 + chunk]
            if bool(zr.any()):
                assert torch.count_nonzero(a_[zr]).item() == 0
    print(f"[bwd] full size: worst {worst} ulp, {exact / total:.4f} bit-identical, "
          f"{int(zero_rows.sum())} zero rows of {N}", flush=True)
    assert worst <= 1
    del x, dl, ref, dlf, xf
    gc.collect()
    torch.cuda.empty_cache()


def _ord(t):
    b = t.view(torch.int16).to(torch.int32)
    return torch.where(b < 0, -(b & 0x7FFF), b)
