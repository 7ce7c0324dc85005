"""MI355X-native pieces of ``rosellm.roseinfer`` on the RoseRLHF path: the
next-token sampler of roseinfer/engine.py:1088-1171, returning the behaviour
log-probabilities that rollout records need (roserlhf/trajectory.py:15,27-28)."""

from .sampling import SampleOutput, sample_next_token, sample_next_token_batch

__all__ = ["SampleOutput", "sample_next_token", "sample_next_token_batch"]
