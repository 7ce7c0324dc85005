"""Next-token sampling kernel (rrl_sample_logprobs) vs the CPU oracle on the
same logits and the same Philox uniforms (MI355X).

Bars: the sampled token equals the oracle's on every row whose uniform lies
farther than 1e-5 of sum(q) from a cumulative boundary (the kernel's float32
partial sums against the oracle's float64 ones); ``logprobs`` within 1e-5
relative (+1e-6) of the float64 log_softmax(x/T) and, at T = 1, of the
training path's own gather_token_logprobs; ``sampling_logprobs`` within 1e-5
relative (+1e-6) of log(q/sum q).  Ties at top-k / top-p thresholds (bf16
logits tie often) resolve lowest index first on both sides.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import sampler_oracle as so
from rosellm_amd import roseinfer as RI
from rosellm_amd import roserlhf as R

pytestmark = pytest.mark.gpu

MARGIN = 1e-5
P_MARGIN = 1e-6  # a top-p cut this close to top_p (in probability) may move by a token


def _check(logits, out, *, temperature, top_k, top_p, do_sample, seed, offset, what):
    x = logits.float().cpu().numpy()
    want = so.sample_rows(x, temperature=temperature, top_k=top_k, top_p=top_p,
                          do_sample=do_sample, seed=seed, offset=offset)
    tok = out.token_ids.cpu().numpy()
    cut = want["p_margin"] > P_MARGIN
    sure = (want["margin"] > MARGIN) & cut
    diff = (tok != want["token"]) & sure
    print(f"{what}: {int(sure.sum())}/{len(tok)} rows decided, {int((~sure).sum())} within "
          f"{MARGIN} of a boundary or {P_MARGIN} of the top-p cut", flush=True)
    assert not diff.any(), (what, np.nonzero(diff)[0][:5], tok[diff][:5], want["token"][diff][:5])
    same = tok == want["token"]
    lp = out.logprobs.cpu().double().numpy()
    err = np.abs(lp - want["logp"])[same]
    assert (err <= 1e-5 * np.abs(want["logp"][same]) + 1e-6).all(), (what, err.max())
    lq = out.sampling_logprobs.cpu().double().numpy()
    sq = same & cut  # log q's normaliser moves with the cut
    errq = np.abs(lq - want["logq"])[sq]
    assert (errq <= 1e-5 * np.abs(want["logq"][sq]) + 1e-6).all(), (what, errq.max())
    return tok


CONFIGS = [
    dict(temperature=1.0, top_k=0, top_p=1.0),     # the reference's defaults
    dict(temperature=0.7, top_k=50, top_p=1.0),
    dict(temperature=1.0, top_k=0, top_p=0.9),
    dict(temperature=1.2, top_k=200, top_p=0.8),
    dict(temperature=1.0, top_k=0, top_p=1e-6),    # first token only (+ floor mass)
]


@pytest.mark.parametrize("dtype,V", [(torch.bfloat16, 151936), (torch.float32, 50257),
                                     (torch.float16, 32000)])
@pytest.mark.parametrize("cfg", CONFIGS, ids=lambda c: f"T{c['temperature']}-k{c['top_k']}-p{c['top_p']}")
def test_sampler_matches_oracle(device, dtype, V, cfg):
    print(f"[sampler] dtype={dtype} V={V} cfg={cfg}", flush=True)
    g = torch.Generator().manual_seed(21)
    B = 48
    x = torch.randn(B, V, generator=g) * 3.0
    hot = torch.randint(0, V, (B,), generator=g)
    x[torch.arange(0, B, 5), hot[::5]] += 15.0  # dominant rows, as config 2
    x = x.to(dtype)
    xd = x.to(device)
    out = RI.sample_next_token_batch(xd, do_sample=True, seed=1234, offset=3, **cfg)
    assert out.token_ids.dtype == torch.int64 and out.logprobs.dtype == torch.float32
    tok = _check(x, out, do_sample=True, seed=1234, offset=3, what=f"{dtype} V={V}", **cfg)
    if cfg["temperature"] == 1.0:
        # the trainer's own recomputation of the same token's log-prob
        lp = R.gather_token_logprobs(xd, out.token_ids).cpu().double()
        got = out.logprobs.cpu().double()
        assert torch.allclose(got, lp, rtol=1e-6, atol=1e-6), (got - lp).abs().max()
    assert (tok >= 0).all() and (tok < V).all()


def test_sampler_ties_at_thresholds(device):
    """bf16 logits on a coarse grid: the top-k and top-p thresholds cut
    through groups of equal logits; eight offsets per row."""

    g = torch.Generator().manual_seed(22)
    B, V = 32, 4096
    x = (torch.round(torch.randn(B, V, generator=g) * 2.0) / 2.0).to(torch.bfloat16)
    xd = x.to(device)
    for cfg in (dict(temperature=1.0, top_k=37, top_p=1.0),
                dict(temperature=1.0, top_k=0, top_p=0.3),
                dict(temperature=0.9, top_k=300, top_p=0.6)):
        for off in range(8):
            out = RI.sample_next_token_batch(xd, do_sample=True, seed=77, offset=off, **cfg)
            _check(x, out, do_sample=True, seed=77, offset=off, what=f"ties {cfg} off={off}", **cfg)


def test_greedy_and_temperature_zero(device):
    g = torch.Generator().manual_seed(23)
    x = (torch.randn(16, 151936, generator=g) * 3.0).to(torch.bfloat16)
    x[3, 10] = x[3].max()  # a tie at the maximum: lowest index wins
    xd = x.to(device)
    for kw in (dict(do_sample=False, temperature=1.0), dict(do_sample=True, temperature=0.0)):
        out = RI.sample_next_token_batch(xd, top_k=5, top_p=0.5, **kw)
        assert torch.equal(out.token_ids.cpu(), torch.argmax(x.float(), dim=-1))
        assert (out.sampling_logprobs == 0).all()
        lp = R.gather_token_logprobs(xd, out.token_ids).cpu()
        assert torch.allclose(out.logprobs.cpu(), lp, rtol=1e-6, atol=1e-6)
    assert RI.sample_next_token(xd[:1], 1.0, 0, 1.0, False) == int(torch.argmax(x[0].float()))


def test_draws_follow_the_distribution(device):
    """8192 draws from one row (rows of a stride-0 view take distinct counters)."""

    V, B = 64, 8192
    g = torch.Generator().manual_seed(24)
    row = torch.randn(V, generator=g) * 1.5
    xd = row.to(device)[None].expand(B, V)
    out = RI.sample_next_token_batch(xd, 1.0, 0, 0.95, True, seed=5)
    q, _ = so.sampling_distribution(row.double().numpy(), 1.0, 0, 0.95)
    counts = np.bincount(out.token_ids.cpu().numpy(), minlength=V)
    expect = q / q.sum() * B
    big = expect > 5
    chi2 = float((((counts[big] - expect[big]) ** 2) / expect[big]).sum())
    dof = int(big.sum()) - 1
    assert chi2 < dof + 6 * np.sqrt(2 * dof), (chi2, dof)
    assert counts[~big].sum() <= max(10, 5 * expect[~big].sum())


def test_bad_rows_and_shapes(device):
    x = torch.randn(4, 100, device=device)
    x[2, 7] = float("nan")
    with pytest.raises(RuntimeError, match="inf"):
        RI.sample_next_token_batch(x, 1.0, 0, 1.0, True, seed=1)
    x[2, 7] = float("inf")
    with pytest.raises(RuntimeError, match="inf"):
        RI.sample_next_token_batch(x, 1.0, 0, 1.0, True, seed=1)
    with pytest.raises(ValueError, match="2D"):
        RI.sample_next_token_batch(x[0], 1.0, 0, 1.0, True)
    empty = RI.sample_next_token_batch(torch.randn(0, 100, device=device), 1.0, 0, 1.0, True)
    assert empty.token_ids.numel() == 0


def _rows(seed, B, V, dtype, scale=3.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, V, generator=g) * scale
    hot = torch.randint(0, V, (B,), generator=g)
    x[torch.arange(0, B, 4), hot[::4]] += 15.0  # dominant rows
    x[1, V // 3] = x[1].max()  # a tie at the maximum (lowest index wins)
    return x.to(dtype)


@pytest.mark.parametrize("dtype,V", [
    (torch.bfloat16, 151936),  # 19 slabs of the 20-slab variant, last one partial
    (torch.bfloat16, 163840),  # 20 whole slabs
    (torch.float16, 65536),    # 8 whole slabs
    (torch.bfloat16, 50264),   # 7 slabs, last one partial
    (torch.bfloat16, 98296),   # 12 slabs of the 12-slab variant, last one partial
    (torch.float16, 128256),   # 16 slabs of the 16-slab variant (Llama-3's vocabulary)
    (torch.float16, 20000),    # 3 slabs, 451 lanes of the last
    (torch.bfloat16, 8),       # one vector
])
@pytest.mark.parametrize("kw", [
    dict(temperature=1.0, top_k=0, top_p=1.0, do_sample=True),
    dict(temperature=0.7, top_k=0, top_p=1.0, do_sample=True),
    dict(temperature=1.0, top_k=0, top_p=1.0, do_sample=False),
    dict(temperature=0.7, top_k=50, top_p=1.0, do_sample=True),
    dict(temperature=1.2, top_k=200, top_p=0.8, do_sample=True),
    dict(temperature=1.0, top_k=1000, top_p=0.95, do_sample=True),
], ids=lambda c: f"T{c['temperature']}-k{c['top_k']}-p{c['top_p']}-s{int(c['do_sample'])}")
def test_resident_rows_match_oracle_and_streamed(device, dtype, V, kw):
    """Whole-vector, 16-byte aligned 16-bit rows are held in registers for
    plain sampling, greedy decoding and top-k (with or without top-p); the
    same logits one element off a 16-byte boundary take the streaming kernel.
    Both follow the oracle, and each other on every row whose uniform is
    decided."""

    print(f"[sampler] resident dtype={dtype} V={V} {kw}", flush=True)
    B = 40
    x = _rows(31 + V % 97, B, V, dtype)
    temperature, do_sample = kw["temperature"], kw["do_sample"]
    xd = x.to(device)
    wide = torch.zeros(B, V + 8, dtype=dtype, device=device)
    wide[:, 1:V + 1] = xd
    for off in (0, 1):
        res = RI.sample_next_token_batch(xd, seed=99, offset=off, **kw)
        st = RI.sample_next_token_batch(wide[:, 1:V + 1], seed=99, offset=off, **kw)
        tok = _check(x, res, seed=99, offset=off, what=f"resident V={V} off={off}", **kw)
        _check(x, st, seed=99, offset=off, what=f"streamed V={V} off={off}", **kw)
        want = so.sample_rows(x.float().numpy(), seed=99, offset=off, **kw)
        sure = (want["margin"] > MARGIN) & (want["p_margin"] > P_MARGIN)
        assert (tok[sure] == st.token_ids.cpu().numpy()[sure]).all()
        if temperature == 1.0:
            lp = R.gather_token_logprobs(xd, res.token_ids).cpu().double()
            assert torch.allclose(res.logprobs.cpu().double(), lp, rtol=1e-6, atol=1e-6)
        if not do_sample:
            assert torch.equal(res.token_ids.cpu(), torch.argmax(x.float(), dim=-1))
            assert (res.sampling_logprobs == 0).all()


@pytest.mark.parametrize("top_k,top_p", [(10, 1.0), (600, 0.9)])
def test_resident_topk_list_overflow(device, top_k, top_p):
    """Rows whose entries at or above the k-th largest lane maximum exceed the
    1024-entry list (here 2000 copies of the maximum, or coarse logits) take
    the streaming row path inside the register-resident launch; the other
    rows of the batch stay in registers.  All follow the oracle."""

    B, V = 12, 32768
    g = torch.Generator().manual_seed(41)
    x = torch.randn(B, V, generator=g) * 3.0
    x[0, torch.randperm(V, generator=g)[:2000]] = 20.0   # 2000 tied maxima
    x[3] = torch.round(x[3] * 2.0) / 2.0                 # coarse grid: many ties
    x[5, 7] = 30.0
    x = x.to(torch.bfloat16)
    kw = dict(temperature=1.0, top_k=top_k, top_p=top_p, do_sample=True)
    for off in range(3):
        out = RI.sample_next_token_batch(x.to(device), seed=13, offset=off, **kw)
        _check(x, out, seed=13, offset=off, what=f"overflow k={top_k} off={off}", **kw)


@pytest.mark.parametrize("top_k,top_p", [(700, 1.0), (900, 0.9), (1024, 1.0)])
def test_resident_topk_exact_kth_relist(device, top_k, top_p):
    """top_k in the hundreds: the entries at or above the k-th largest lane
    maximum overflow the 1024-entry list into its 3072-entry tail, so the
    kernel takes the exact k-th key over all of them and keeps the entries at
    or above it.  Rows: N(0, 3), a spike of 4000, a grid of quarters (ties at
    the k-th key: past 1024 entries at top_k 1024, the streaming path),
    N(0, 1)."""

    B, V = 6, 151936
    g = torch.Generator().manual_seed(43)
    x = torch.randn(B, V, generator=g) * 3.0
    x[1, 11] = 4000.0
    x[2] = torch.round(x[2] * 4.0) / 4.0                 # quarters: ties
    x[4] = x[4] / 3.0
    x = x.to(torch.bfloat16)
    kw = dict(temperature=1.0, top_k=top_k, top_p=top_p, do_sample=True)
    for off in range(2):
        out = RI.sample_next_token_batch(x.to(device), seed=17, offset=off, **kw)
        _check(x, out, seed=17, offset=off, what=f"relist k={top_k} off={off}", **kw)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("top_k,top_p", [(100, 0.305), (400, 0.7537), (90, 0.999)])
def test_long_list_top_p_ties(device, dtype, top_k, top_p):
    """Lists of 65-1024 candidates with many equal keys: logits on a grid of
    halves, so the k-th key and top-p's threshold group each hold many tied
    entries (kept lowest index first, the group cut by its equal masses).
    16-bit rows take the register-resident list path (counting sort, radix
    select, mass histograms); float32 rows the streaming kernel's list with
    32-bit keys; row 2's 5002 tied maxima the streaming path.  top_p is kept
    off exact multiples of a tied group's probability (0.3 = 30 x 0.01
    exactly: the kernels' fixed-point cut keeps 30 there, the oracle's
    float64 cumsum, 0.30000000000000004 > 0.3, keeps 29)."""

    B, V = 8, 40000
    g = torch.Generator().manual_seed(47)
    x = torch.round(torch.randn(B, V, generator=g) * 4.0) / 2.0
    x[1] = torch.round(x[1])                              # coarser: more ties
    x[2, :5000] = x[2].max()                              # tied maxima past the list
    x = x.to(dtype)
    kw = dict(temperature=1.0, top_k=top_k, top_p=top_p, do_sample=True)
    for off in range(3):
        out = RI.sample_next_token_batch(x.to(device), seed=19, offset=off, **kw)
        _check(x, out, seed=19, offset=off, what=f"ties {dtype} k={top_k} p={top_p} off={off}", **kw)


@pytest.mark.parametrize("V", [
    151936,  # 19 slabs of the 20-slab variant, last one partial
    128256,  # 16 whole slabs
    98296,   # 12 slabs, last one partial
    50264,   # 7 slabs of the 8-slab variant, last one partial
    20000,   # 3 slabs of the 4-slab variant, 451 lanes of the last
])
@pytest.mark.parametrize("top_p", [0.5, 0.9, 0.999])
def test_resident_nucleus_rows(device, top_p, V):
    """top_p without top-k on bfloat16 rows: counts per key from the cut's
    lower bound up in registers.  Rows: N(0, 3); a dominant token; ties on a
    grid of halves (the threshold group's lowest indices kept); a flat row of
    N(0, 0.01), whose keys from the lower bound up span most binades near
    zero, so the row is handed to the fill-in launch of the streaming kernel
    (token slot -1 in between); ties on a grid of quarters; an all-negative
    row (log-probs: every counted key a negative number's, the other form of
    the slot arithmetic)."""

    B = 8
    g = torch.Generator().manual_seed(53)
    x = torch.randn(B, V, generator=g) * 3.0
    x[1, 777] += 25.0
    x[2] = torch.round(x[2] * 2.0) / 2.0
    x[3] = torch.randn(V, generator=g) * 0.01
    x[5] = torch.round(x[5]) / 4.0
    x[6] = torch.log_softmax(x[6], dim=0)
    x = x.to(torch.bfloat16)
    assert float(x[6].float().max()) < 0.0
    # The hand-over is decided by the number of bfloat16 keys from the cut's
    # lower bound x_lo up to the row maximum: more than the kernel's 4096
    # counts sends the row to the fill-in launch.  Recomputed here with the
    # kernel's formula: the flat row 3 lies far beyond (about 32000 keys), the
    # N(0, 3) row 0 far inside when x_lo stays above zero (top_p 0.5, 0.9),
    # and so does the all-negative row 6.
    spans = [_nucleus_key_span(x[i], top_p) for i in range(B)]
    print(f"[sampler] nucleus V={V} p={top_p}: keys from x_lo up per row {spans}", flush=True)
    assert spans[3] >= 2 * 4096, "row 3 no longer reaches the fill-in launch"
    assert spans[6] <= 4096 // 2, "row 6 no longer takes the resident nucleus path"
    if top_p < 0.99 and V >= 50000:
        assert spans[0] <= 4096 // 2, "row 0 no longer takes the resident nucleus path"
    kw = dict(temperature=1.0, top_k=0, top_p=top_p, do_sample=True)
    for off in range(3):
        out = RI.sample_next_token_batch(x.to(device), seed=23, offset=off, **kw)
        tok = _check(x, out, seed=23, offset=off, what=f"nucleus V={V} p={top_p} off={off}",
                     **kw)
        assert (tok >= 0).all() and (tok < V).all()


def _bf16_key(v):
    """The kernels' ordered 16-bit key of a value rounded toward zero to
    bfloat16 (float_key: +-0 share a key; negative values below positive)."""

    b = (int(torch.tensor([v], dtype=torch.float32).view(torch.int32).item()) >> 16) & 0xFFFF
    if b & 0x7FFF == 0:
        b = 0
    return (~b & 0xFFFF) if b & 0x8000 else (b | 0x8000)


def _nucleus_key_span(row, top_p, temperature=1.0):
    """kmax - klo of the resident nucleus path for one bfloat16 row: x_lo =
    M + log2((1 - top_p) Z / (2 V)) / c2 with Z = sum 2^((x - M) c2) and c2 =
    log2(e) / T; klo is one key below x_lo's."""

    r = row.double()
    V = r.numel()
    M = float(r.max())
    c2 = math.log2(math.e) / temperature
    Z = float(torch.exp2((r - M) * c2).sum())
    xlo = M + math.log2((1.0 - top_p) * Z / (2.0 * V)) / c2
    return _bf16_key(M) - max(_bf16_key(xlo) - 1, 0)


@pytest.mark.parametrize("case", ["spike", "cold", "masked_head"])
@pytest.mark.parametrize("do_sample", [True, False])
def test_block_sums_against_far_references(device, case, do_sample):
    """Plain sampling and greedy decoding sum each wave's 512-entry block of a
    slab against the maximum of that wave's block of slab 0; a wave whose
    reference lies more than 64 binary orders below the row maximum redoes its
    sums against the maximum.  Rows that take that path: a spike of +80 (half
    the rows in slab 0, half later) over N(0, 1) logits at T = 1; N(0, 3)
    logits at T = 0.08; a vocabulary head of 10000 entries masked to -inf, so
    that every wave's block of slab 0 is empty."""

    B, V = 24, 151936
    g = torch.Generator().manual_seed(77)
    x = torch.randn(B, V, generator=g)
    T = 1.0
    if case == "spike":
        rows = torch.arange(B)
        at = torch.where(rows % 2 == 0, 97 * rows, 20000 + 5003 * rows)
        x[rows, at] = 80.0
    elif case == "cold":
        x *= 3.0
        T = 0.08
    else:
        x *= 3.0
        x[:, :10000] = float("-inf")
    x = x.to(torch.bfloat16)
    kw = dict(temperature=T, top_k=0, top_p=1.0, do_sample=do_sample)
    print(f"[sampler] far references case={case} {kw}", flush=True)
    xd = x.to(device)
    for off in (0, 3):
        out = RI.sample_next_token_batch(xd, seed=5, offset=off, **kw)
        _check(x, out, seed=5, offset=off, what=f"{case} off={off}", **kw)
        if T == 1.0:
            lp = R.gather_token_logprobs(xd, out.token_ids).cpu().double()
            assert torch.allclose(out.logprobs.cpu().double(), lp, rtol=1e-6, atol=1e-6)
        if not do_sample:
            assert torch.equal(out.token_ids.cpu(), torch.argmax(x.float(), dim=-1))


# (seed, row) pairs at offset 0 whose component uniform u1 lies below
# V * 1e-9 for V = 8192, found by a search over seeds with the oracle's Philox.
FLOOR_HITS = [(9715, 7), (15203, 4), (38829, 0)]


@pytest.mark.parametrize("seed,row", FLOOR_HITS)
@pytest.mark.parametrize("layout", ["resident", "streamed"])
def test_floor_excess_component(device, seed, row, layout):
    """The rare side of the mixture: rows whose component uniform falls below
    V * 1e-9, where the kernels total the floor's excess G and draw from
    max(1e-9 - p, 0) when u1 < G / (1 + G).  Row `row` is made almost
    entirely floored (a spike of +30 over N(0, 1): G = (V - 1) 1e-9, the
    excess is drawn), then half floored (4095 entries at 12, 4096 near 0:
    G = 4096e-9, so u1 of the first two seeds lies between G / (1 + G) and
    V * 1e-9 and p is drawn after all).  Both kernels against the oracle;
    the excess's weights are near-uniform over thousands of entries, so the
    decisions are far from any boundary."""

    V, B = 8192, 16
    u, u1 = so.row_uniforms(seed, 0, row)
    assert u1 < V * 1e-9
    g = torch.Generator().manual_seed(seed)
    for shape in ("floored", "half"):
        x = torch.randn(B, V, generator=g) * 3.0
        x[row] = torch.randn(V, generator=g)
        if shape == "half":
            x[row, : V // 2] += 12.0
        x[row, 1234] = 30.0
        x = x.to(torch.bfloat16)
        p = torch.softmax(x[row].double(), dim=0).numpy()
        _, gx, pi = so.mixture_parts(p)
        print(f"[sampler] floor excess seed={seed} row={row} {layout} {shape}: u1={u1:.3e} "
              f"G/(1+G)={pi:.3e}", flush=True)
        xd = x.to(device)
        if layout == "streamed":  # one element off a 16-byte boundary
            wide = torch.zeros(B, V + 8, dtype=x.dtype, device=device)
            wide[:, 1:V + 1] = xd
            xd = wide[:, 1:V + 1]
        kw = dict(temperature=1.0, top_k=0, top_p=1.0, do_sample=True)
        out = RI.sample_next_token_batch(xd, seed=seed, offset=0, **kw)
        tok = _check(x, out, seed=seed, offset=0, what=f"floor {shape} {layout}", **kw)
        want = so.sample_rows(x.float().numpy(), seed=seed, offset=0, **kw)
        assert want["margin"][row] > MARGIN
        # the excess was drawn exactly when u1 < G / (1 + G): a floored token
        assert (gx[tok[row]] > 0) == (u1 < pi), (shape, tok[row], u1, pi)


@pytest.mark.parametrize("kw", [
    dict(temperature=1.0, top_k=0, top_p=1.0, do_sample=True),
    dict(temperature=0.7, top_k=50, top_p=0.9, do_sample=True),
    dict(temperature=1.0, top_k=0, top_p=1.0, do_sample=False),
], ids=["defaults", "topk-topp", "greedy"])
def test_without_sampling_logprobs(device, kw):
    """sampling_logprobs=False leaves the token and log-prob of every row as
    they are (the same uniforms, the same draw) and returns no log q."""

    x = _rows(5, 32, 151936, torch.bfloat16).to(device)
    full = RI.sample_next_token_batch(x, seed=21, offset=4, **kw)
    bare = RI.sample_next_token_batch(x, seed=21, offset=4, sampling_logprobs=False, **kw)
    assert bare.sampling_logprobs is None
    assert torch.equal(bare.token_ids, full.token_ids)
    assert torch.equal(bare.logprobs, full.logprobs)


def test_resident_draws_follow_the_distribution(device):
    """8192 draws from one bf16 row held in registers (a stride-0 view)."""

    V, B = 64, 8192
    g = torch.Generator().manual_seed(25)
    row = (torch.randn(V, generator=g) * 1.5).to(torch.bfloat16)
    xd = row.to(device)[None].expand(B, V)
    out = RI.sample_next_token_batch(xd, 1.0, 0, 1.0, True, seed=6)
    q, _ = so.sampling_distribution(row.double().numpy(), 1.0, 0, 1.0)
    counts = np.bincount(out.token_ids.cpu().numpy(), minlength=V)
    expect = q / q.sum() * B
    big = expect > 5
    chi2 = float((((counts[big] - expect[big]) ** 2) / expect[big]).sum())
    dof = int(big.sum()) - 1
    assert chi2 < dof + 6 * np.sqrt(2 * dof), (chi2, dof)


@pytest.mark.parametrize("bad", ["nan", "nan_after_inf", "inf", "all_neg_inf"])
@pytest.mark.parametrize("dtype,V", [(torch.bfloat16, 4096), (torch.float32, 4099)])
def test_bad_rows_sampling_raises_greedy_is_argmax(device, bad, dtype, V):
    """Sampling raises on a row with NaN / +inf / no finite logit, as
    torch.multinomial does; greedy decoding is torch.argmax in the reference
    (engine.py:1117-1118), which never raises: the bad row keeps argmax's token
    (the first NaN, else the first maximum) and gets a NaN log-prob.  bf16 rows
    of whole vectors take the register-resident kernel, V = 4099 float32 rows
    the streaming one."""

    x = torch.randn(4, V, device=device).to(dtype)
    if bad == "nan":
        x[2, 4000] = float("nan")
        x[2, 4001] = float("nan")
    elif bad == "nan_after_inf":
        x[2, 9] = float("inf")
        x[2, 3000] = float("nan")
    elif bad == "inf":
        x[2, 7] = float("inf")
        x[2, 70] = float("inf")
    else:
        x[2] = -float("inf")
    with pytest.raises(RuntimeError, match="inf"):
        RI.sample_next_token_batch(x, 1.0, 0, 1.0, True, seed=1)
    for temperature, do_sample in ((1.0, False), (0.0, True)):
        out = RI.sample_next_token_batch(x, temperature, 0, 1.0, do_sample, seed=1)
        assert torch.equal(out.token_ids.cpu(), torch.argmax(x.cpu(), dim=-1))
        lp = out.logprobs.cpu()
        assert torch.isnan(lp[2]) and torch.isfinite(lp[[0, 1, 3]]).all()
    # the other rows of a call are unaffected when run alone
    ok = RI.sample_next_token_batch(x[:2], 1.0, 0, 1.0, False)
    assert torch.equal(ok.token_ids.cpu(), torch.argmax(x[:2].float(), dim=-1).cpu())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_bad_rows_through_the_c_abi(device, dtype):
    """The status word gets BAD_PROBS and the bad row's log-probs are NaN,
    the others finite (register-resident bf16 rows and streamed float32
    rows); -3e38 logits at T = 0.5 overflow x / T and count as bad."""

    from rosellm_amd import _native as nat

    B, V = 4, 4096
    x = torch.randn(B, V, device=device).to(dtype)
    x[1, 100] = float("nan")
    x[3] = -3.0e38
    for temperature, do_sample in ((0.5, 1), (1.0, 0)):
        tok = torch.empty(B, dtype=torch.int64, device=device)
        lp = torch.empty(B, device=device)
        lq = torch.empty(B, device=device)
        st = torch.zeros(1, dtype=torch.int32, device=device)
        nat.call("rrl_sample_logprobs", x.data_ptr(), nat.dtype_code(dtype), B, V, V,
                 temperature, 0, 1.0, do_sample, 3, 0, tok.data_ptr(), lp.data_ptr(),
                 lq.data_ptr(), st.data_ptr(), nat.stream_ptr(device))
        flagged = int(st.item()) & nat.FLAG_BAD_PROBS
        bad = torch.isnan(lp).cpu()
        want_bad = torch.tensor([False, True, False, temperature < 1.0])
        assert torch.equal(bad, want_bad), (temperature, bad)
        assert bool(flagged)
        assert torch.isnan(lq.cpu()[want_bad]).all() and torch.isfinite(lp.cpu()[~want_bad]).all()
        if not do_sample:
            assert torch.equal(tok.cpu(), torch.argmax(x.cpu(), dim=-1))


@pytest.mark.parametrize("dtype,misaligned", [(torch.bfloat16, False), (torch.bfloat16, True),
                                              (torch.float32, False)])
def test_signed_zero_ties(device, dtype, misaligned):
    """-0.0 and +0.0 compare equal: at a top-k or top-p threshold that falls
    among zeros of both signs they form one group of ties, kept lowest index
    first, in the register-resident and the streaming kernel alike."""

    g = torch.Generator().manual_seed(51)
    B, V = 16, 4096
    x = torch.randn(B, V, generator=g) - 2.0
    zero = torch.rand(B, V, generator=g) < 0.2
    neg = torch.rand(B, V, generator=g) < 0.5
    x = torch.where(zero, torch.where(neg, torch.tensor(-0.0), torch.tensor(0.0)), x)
    x[:, :16] = torch.rand(B, 16, generator=g) + 0.5  # a few entries above the zeros
    assert bool((torch.signbit(x) & (x == 0)).any()) and bool((~torch.signbit(x) & (x == 0)).any())
    x = x.to(dtype)
    if misaligned:
        wide = torch.zeros(B, V + 8, dtype=dtype, device=device)
        wide[:, 1:V + 1] = x.to(device)
        xd = wide[:, 1:V + 1]
    else:
        xd = x.to(device)
    for k, p in ((100, 1.0), (0, 0.5), (400, 0.5), (900, 0.5)):
        kw = dict(temperature=1.0, top_k=k, top_p=p, do_sample=True)
        for off in range(3):
            out = RI.sample_next_token_batch(xd, seed=17, offset=off, **kw)
            _check(x, out, seed=17, offset=off, what=f"signed zeros k={k} p={p} off={off}", **kw)



@pytest.mark.parametrize("V", [151936, 50264])
@pytest.mark.parametrize("temperature", [1.0, 0.7])
def test_floor_excess_regimes(device, V, temperature):
    """The reference's defaults (top_k 0, top_p 1) with log q on rows whose
    floor excess G comes from very different parts of the row: N(0, 3)
    (entries below -4 floored at T 1), shifted by +30 and +45 (the floored
    band among large positive logits), a dominant token, log-probs (every
    logit negative), and a third of a row pushed 40 down (thousands of
    entries floored outright).  log q against the oracle's float64 value."""

    B = 8
    g = torch.Generator().manual_seed(71)
    x = torch.randn(B, V, generator=g) * 3.0
    x[1] += 30.0
    x[2, 4321] += 25.0
    x[3] = torch.log_softmax(x[3], dim=0)
    x[4] = torch.randn(V, generator=g) * 3.0 + 45.0
    x[5, : V // 3] -= 40.0
    x = x.to(torch.bfloat16)
    kw = dict(temperature=temperature, top_k=0, top_p=1.0, do_sample=True)
    for off in range(3):
        out = RI.sample_next_token_batch(x.to(device), seed=29, offset=off, **kw)
        _check(x, out, seed=29, offset=off, what=f"excess V={V} T={temperature} off={off}", **kw)
