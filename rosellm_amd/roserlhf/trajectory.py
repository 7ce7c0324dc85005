"""Immutable trajectory records of the RoseRLHF rollout side
(rosellm/roserlhf/trajectory.py:9-102): the same classes, fields, defaults,
validation rules and messages, so records built for the reference load here
unchanged.  Plain host-side Python: these hold token ids and behaviour
log-probs exactly as sampled; ``rosellm_amd.roserlhf.packing`` turns them into
the [B, L] tensors the kernels consume."""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Sequence

__all__ = ["PolicyAction", "TransitionRecord", "Trajectory"]


@dataclass(frozen=True)
class PolicyAction:
    """The tokens one behaviour policy sampled for one turn, with the
    log-probability of each (trajectory.py:9-31)."""

    turn: int
    token_ids: Sequence[int]
    old_logprobs: Sequence[float]
    policy_version: str
    text: str
    parsed_action: Optional[Dict[str, Any]] = None

    def __post_init__(self) -> None:
        checks = (
            (self.turn < 0, "turn must be non-negative"),
            (not self.policy_version, "policy_version is required"),
            (len(self.token_ids) == 0, "a policy action must contain at least one token"),
            (len(self.token_ids) != len(self.old_logprobs),
             "every sampled token needs its behavior log-probability"),
            (any(t < 0 for t in self.token_ids), "token IDs must be non-negative"),
        )
        for failed, message in checks:
            if failed:
                raise ValueError(message)


@dataclass(frozen=True)
class TransitionRecord:
    """What the environment returned after a turn's action (trajectory.py:34-50)."""

    turn: int
    observation_ref: str
    reward_components: Dict[str, float] = field(default_factory=dict)
    terminated: bool = False
    truncated: bool = False
    state_hash: Optional[str] = None

    def __post_init__(self) -> None:
        if self.turn < 0:
            raise ValueError("turn must be non-negative")
        if not self.observation_ref:
            raise ValueError("observation_ref is required")
        if self.terminated and self.truncated:
            raise ValueError("a transition cannot be both terminated and truncated")


@dataclass
class Trajectory:
    """One task attempt: action/transition pairs in turn order
    (trajectory.py:53-102)."""

    trajectory_id: str
    task_id: str
    environment_version: str
    tokenizer_hash: str
    actions: List[PolicyAction] = field(default_factory=list)
    transitions: List[TransitionRecord] = field(default_factory=list)

    def append(self, action: PolicyAction, transition: TransitionRecord) -> None:
        if self.is_finished:
            raise ValueError("cannot append to a finished trajectory")
        turn = len(self.actions)
        if (action.turn, transition.turn) != (turn, turn):
            raise ValueError(f"expected turn {turn}")
        self.actions.append(action)
        self.transitions.append(transition)

    @property
    def is_finished(self) -> bool:
        if not self.transitions:
            return False
        last = self.transitions[-1]
        return last.terminated or last.truncated

    @property
    def behavior_policy_versions(self) -> List[str]:
        """Distinct behaviour policy versions, first-seen order."""

        seen: Dict[str, None] = {}
        for a in self.actions:
            seen.setdefault(a.policy_version, None)
        return list(seen)

    def validate(self, *, require_finished: bool = True) -> None:
        if not (self.trajectory_id and self.task_id):
            raise ValueError("trajectory_id and task_id are required")
        if not (self.environment_version and self.tokenizer_hash):
            raise ValueError("environment_version and tokenizer_hash are required")
        if len(self.actions) != len(self.transitions):
            raise ValueError("every action must have one transition")
        last = len(self.transitions) - 1
        for i, (a, tr) in enumerate(zip(self.actions, self.transitions)):
            if a.turn != i or tr.turn != i:
                raise ValueError("turns must be contiguous and ordered")
            if i < last and (tr.terminated or tr.truncated):
                raise ValueError("no events may follow a terminal/truncated transition")
        if require_finished and not self.is_finished:
            raise ValueError("trajectory is incomplete")
