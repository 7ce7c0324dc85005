"""MI355X-native RoseRLHF hot path: same public names as ``rosellm.roserlhf``
(rosellm/roserlhf/__init__.py:8-48), backed by gfx950 HIP kernels.

``fused_policy_loss``, ``fused_linear_policy_loss``, ``linear_token_logprobs``,
``masked_whiten`` and ``pack_trajectories`` are additions of this package;
the record types live in ``rosellm_amd.roserlhf.trajectory`` as in the
reference (rosellm/roserlhf/trajectory.py);
``losses.masked_mean`` and ``losses.sequence_log_ratio`` stay module-level as
in the reference.
"""

from .advantages import (
    broadcast_turn_advantages,
    discounted_returns,
    generalized_advantage_estimation,
    group_standardized_advantages,
    leave_one_out_advantages,
    masked_whiten,
    skip_observation_generalized_advantage_estimation,
)
from .linear import fused_linear_policy_loss, linear_token_logprobs
from .packing import PackedTrajectories, pack_trajectories
from .losses import (
    GspoPolicyLossOutput,
    PolicyLossOutput,
    SapoPolicyLossOutput,
    SaoPolicyLossOutput,
    clipped_policy_loss,
    direct_double_sided_mask,
    fused_policy_loss,
    gather_token_logprobs,
    gspo_policy_loss,
    gspo_token_policy_loss,
    sapo_policy_loss,
    sao_policy_loss,
)

__all__ = [
    "GspoPolicyLossOutput",
    "PackedTrajectories",
    "PolicyLossOutput",
    "SapoPolicyLossOutput",
    "SaoPolicyLossOutput",
    "broadcast_turn_advantages",
    "clipped_policy_loss",
    "discounted_returns",
    "direct_double_sided_mask",
    "fused_linear_policy_loss",
    "fused_policy_loss",
    "gather_token_logprobs",
    "generalized_advantage_estimation",
    "group_standardized_advantages",
    "leave_one_out_advantages",
    "linear_token_logprobs",
    "gspo_policy_loss",
    "gspo_token_policy_loss",
    "masked_whiten",
    "pack_trajectories",
    "sapo_policy_loss",
    "sao_policy_loss",
    "skip_observation_generalized_advantage_estimation",
]
