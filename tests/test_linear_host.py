"""Host side of the matrix-core LM-head path, without a GPU: the argument
validation that runs before any device work, and no CPU fallback."""

from __future__ import annotations

import pytest
import torch

from rosellm_amd import roserlhf as R


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
        R.linear_token_logprobs(h, w, t, row_block=0)
    with pytest.raises(ValueError, match="unknown impl"):
        R.linear_token_logprobs(h, w, t, impl="cublas")
    # the tile path's own limits are checked on the host, before any device work
    with pytest.raises(TypeError, match="bfloat16"):
        R.fused_linear_policy_loss(h, w, t, z, z, z.bool(), impl="tiles")
    hb, wb = h.bfloat16(), w.bfloat16()
    with pytest.raises(ValueError, match="multiple of 128"):
        R.linear_token_logprobs(hb, wb, t, impl="tiles")


def test_no_cpu_fallback():
    h = torch.zeros(2, 3, 8)
    w = torch.zeros(11, 8)
    t = torch.zeros(2, 3, dtype=torch.long)
    z = torch.zeros(2, 3)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        R.fused_linear_policy_loss(h, w, t, z, z, z.bool())
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        R.fused_linear_policy_loss(h, w, t, z, z, z.bool(), skip_masked_rows=True)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        R.linear_token_logprobs(h, w, t)
