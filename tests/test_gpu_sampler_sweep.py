"""Seeded random sweep of the next-token sampler against the CPU oracle
(MI355X): bf16, f16 and float32 rows; vocabularies from 1 to 163840 entries
(whole and partial slabs, V % 8 != 0); contiguous, row-strided, stride-0 and
16-byte-misaligned views; greedy decoding, temperature, top-k (short lists,
lists of 65-1024 entries, gathers into the list's tail and lists that overflow
into the streaming path), top-p and both together; peaked,
flat and coarse (tie-heavy) logits.  Every call takes one of the two kernels
(register-resident or streaming) by its shape and settings, so the sweep holds
both to the oracle.  Bars as in test_gpu_sampler: tokens equal wherever the
uniform is decided (1e-5 of the total away from a boundary), log-probs 1e-5
relative + 1e-6."""

from __future__ import annotations

import random

import pytest
import torch

from rosellm_amd import roseinfer as RI

from test_gpu_sampler import _check

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16, torch.float32]
VOCABS = [1, 2, 8, 9, 64, 1000, 4096, 8192, 20000, 50257, 65536, 98296, 151936, 163840]
SETTINGS = [
    dict(temperature=1.0, top_k=0, top_p=1.0, do_sample=True),
    dict(temperature=0.6, top_k=0, top_p=1.0, do_sample=True),
    dict(temperature=1.0, top_k=0, top_p=1.0, do_sample=False),
    dict(temperature=1.0, top_k=20, top_p=1.0, do_sample=True),
    dict(temperature=0.8, top_k=700, top_p=0.95, do_sample=True),
    dict(temperature=1.3, top_k=0, top_p=0.7, do_sample=True),
    dict(temperature=1.0, top_k=1, top_p=1.0, do_sample=True),
    dict(temperature=1.0, top_k=150, top_p=0.8, do_sample=True),
    dict(temperature=0.9, top_k=400, top_p=1.0, do_sample=True),
]


def _case(i):
    rng = random.Random(9100 + i)
    return dict(seed=9100 + i, dtype=DTYPES[i % 3], V=rng.choice(VOCABS),
                setting=SETTINGS[(i // 3) % len(SETTINGS)], B=rng.choice([1, 3, 17, 64]),
                layout=rng.choice(["contiguous", "row_stride", "misaligned", "broadcast"]),
                logits=rng.choice(["peaked", "flat", "coarse"]))


CASES = [_case(i) for i in range(108)]


def _ids(c):
    s = c["setting"]
    return (f"{str(c['dtype'])[6:]}-V{c['V']}-B{c['B']}-{c['layout']}-{c['logits']}-"
            f"T{s['temperature']}-k{s['top_k']}-p{s['top_p']}-s{int(s['do_sample'])}")


@pytest.mark.parametrize("c", CASES, ids=_ids)
def test_sampler_sweep(device, c):
    print(f"[sampler sweep] {_ids(c)}", flush=True)
    g = torch.Generator().manual_seed(c["seed"])
    B, V = c["B"], c["V"]
    if c["logits"] == "peaked":
        x = torch.randn(B, V, generator=g) * 2.0
        x[torch.arange(B), torch.randint(0, V, (B,), generator=g)] += 12.0
    elif c["logits"] == "flat":
        x = torch.randn(B, V, generator=g) * 0.5
    else:
        x = torch.round(torch.randn(B, V, generator=g) * 2.0) / 2.0
    x = x.to(c["dtype"])
    if c["layout"] == "contiguous":
        xd = x.to(device)
    elif c["layout"] == "row_stride":
        wide = torch.zeros(B, V + 24, dtype=c["dtype"], device=device)
        wide[:, :V] = x.to(device)
        xd = wide[:, :V]
    elif c["layout"] == "misaligned":
        wide = torch.zeros(B, V + 8, dtype=c["dtype"], device=device)
        wide[:, 1:V + 1] = x.to(device)
        xd = wide[:, 1:V + 1]
    else:  # every row the same storage (stride 0): distinct uniforms per row
        x = x[:1].expand(B, V).contiguous()
        xd = x[:1].to(device).expand(B, V)
    s = c["setting"]
    out = RI.sample_next_token_batch(xd, seed=c["seed"], offset=5, **s)
    tok = _check(x, out, seed=c["seed"], offset=5, what=_ids(c), **s)
    assert (tok >= 0).all() and (tok < V).all()
