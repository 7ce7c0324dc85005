"""Host side of the fused LM-head path, without a GPU: the row-block
partition and the argument validation that runs before any device work."""

from __future__ import annotations

import pytest
import torch

from rosellm_amd import roserlhf as R
from rosellm_amd.roserlhf import linear as LIN


def _partition(B, T, row_block):
    if T <= row_block:
        bc = max(1, row_block // T)
        return [(b0, min(B, b0 + bc), 0, T) for b0 in range(0, B, bc)]
    return [(b, b + 1, t0, min(T, t0 + row_block)) for b in range(B) for t0 in range(0, T, row_block)]


@pytest.mark.parametrize("B,T,rb", [(8, 96, 64), (8, 96, 192), (8, 96, 4096), (3, 5, 7),
                                    (1, 10, 3), (256, 1024, 16384), (64, 8192, 16384)])
def test_partition_covers_every_row_once(B, T, rb):
    blk = LIN._Blocks(torch.zeros(B * T, 4), torch.zeros(6, 4), B, T, rb)
    assert blk.blocks == _partition(B, T, rb)
    seen = torch.zeros(B * T, dtype=torch.int32)
    for b in blk.blocks:
        r0, n = blk.r0(b), blk.rows(b)
        assert n <= max(rb, T)
        seen[r0:r0 + n] += 1
    assert bool((seen == 1).all())
    assert blk.buf.shape == (max(blk.rows(b) for b in blk.blocks), 6)


def test_validation_messages():
    h = torch.zeros(2, 3, 8)
    w = torch.zeros(11, 8)
    t = torch.zeros(2, 3, dtype=torch.long)
    z = torch.zeros(2, 3)
    with pytest.raises(ValueError, match="unknown objective"):
        R.fused_linear_policy_loss(h, w, t, z, z, z.bool(), objective="dpo")
    with pytest.raises(ValueError, match="weight must be"):
        R.fused_linear_policy_loss(h, torch.zeros(11, 7), t, z, z, z.bool())
    with pytest.raises(TypeError, match="share a dtype"):
        R.fused_linear_policy_loss(h, w.double(), t, z, z, z.bool())
    with pytest.raises(ValueError, match="must match hidden prefix"):
        R.fused_linear_policy_loss(h, w, t[:, :2], z, z, z.bool())
    with pytest.raises(TypeError, match="integer tensor"):
        R.fused_linear_policy_loss(h, w, z, z, z, z.bool())
    with pytest.raises(ValueError, match="all tensors must have the same shape"):
        R.fused_linear_policy_loss(h, w, t, z[:, :2], z, z.bool())
    with pytest.raises(ValueError, match="skip_masked_rows"):
        R.fused_linear_policy_loss(h, w, t, z, z, z.bool(), skip_masked_rows=True,
                                   return_logprobs=True)
    with pytest.raises(ValueError, match="row_block must be positive"):
        LIN._Blocks(torch.zeros(6, 8), w, 2, 3, 0)


def test_no_cpu_fallback():
    h = torch.zeros(2, 3, 8)
    w = torch.zeros(11, 8)
    t = torch.zeros(2, 3, dtype=torch.long)
    z = torch.zeros(2, 3)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        R.fused_linear_policy_loss(h, w, t, z, z, z.bool())
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        R.linear_token_logprobs(h, w, t)
