"""Concurrent calls on two HIP streams (MI355X).

The C ABI promises reentrant calls, ordered on the caller's stream, with no
state shared between calls.  Two host threads run fused_policy_loss (and the
sampler) at the same time, each on its own torch stream (default priority),
on different inputs.  Every result must be bit-identical to the same call run
alone on the default stream.
"""

from __future__ import annotations

import threading

import pytest
import torch

from rosellm_amd import roseinfer as RI
from rosellm_amd import roserlhf as R

pytestmark = pytest.mark.gpu


def _inputs(seed, B, T, V, device):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, T, V, generator=g) * 3.0).to(torch.bfloat16)
    t = torch.randint(0, V, (B, T), generator=g)
    old = torch.randn(B, T, generator=g) * 0.1 - 12.0
    adv = torch.randn(B, T, generator=g)
    mask = torch.rand(B, T, generator=g) < 0.8
    return [v.to(device) for v in (x, t, old, adv, mask)]


def _step(x, t, old, adv, mask):
    xd = x.detach().clone().requires_grad_()
    out, lp = R.fused_policy_loss(xd, t, old, adv, mask, return_logprobs=True,
                                  clip_low=0.2, clip_high=0.28)
    out.loss.backward()
    return out.loss.detach(), lp.detach(), xd.grad


def test_two_streams_match_sequential(device):
    V = 151936
    sets = [_inputs(60 + i, 4, 64, V, device) for i in range(2)]
    logits = [(torch.randn(64, V, device=device) * 3).to(torch.bfloat16) for _ in range(2)]
    want = [_step(*s) for s in sets]
    want_s = [RI.sample_next_token_batch(lg, 1.0, 0, 1.0, True, seed=7, offset=i)
              for i, lg in enumerate(logits)]
    torch.cuda.synchronize()

    got, got_s, errors = [None, None], [None, None], []
    streams = [torch.cuda.Stream(device=device) for _ in range(2)]  # default priority
    start = threading.Barrier(2)

    def worker(i):
        try:
            with torch.cuda.stream(streams[i]):
                start.wait()
                for _ in range(3):
                    got[i] = _step(*sets[i])
                    got_s[i] = RI.sample_next_token_batch(logits[i], 1.0, 0, 1.0, True,
                                                          seed=7, offset=i)
            streams[i].synchronize()
        except Exception as e:  # reported below, never swallowed
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not errors, errors
    torch.cuda.synchronize()
    for i in range(2):
        for a, b in zip(got[i], want[i]):
            assert torch.equal(a, b), i
        assert torch.equal(got_s[i].token_ids, want_s[i].token_ids)
        assert torch.equal(got_s[i].logprobs, want_s[i].logprobs)
        assert torch.equal(got_s[i].sampling_logprobs, want_s[i].sampling_logprobs)
