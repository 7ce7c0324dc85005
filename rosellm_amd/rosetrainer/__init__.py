"""MI355X-native pieces of ``rosellm.rosetrainer`` that sit on the RoseRLHF hot
path's row kernels: the supervised next-token cross-entropy the reference's
model forwards compute (rosetrainer/model.py:643-649,
rosetrainer/qwen3.py:558-564), on logits or straight from the LM head."""

from .lm_loss import (
    causal_lm_loss,
    cross_entropy,
    fused_linear_cross_entropy,
    linear_causal_lm_loss,
)

__all__ = [
    "causal_lm_loss",
    "cross_entropy",
    "fused_linear_cross_entropy",
    "linear_causal_lm_loss",
]
