"""Trajectory records -> the padded token tensors of the training step.

The reference stores rollouts as ``Trajectory`` records
(rosellm/roserlhf/trajectory.py:9-102) and specifies the tensors a training
step consumes (docs/agentic-rl/mathematical-foundations.md:618-640,
training-pipeline.md:309-330) without a function that builds them.  This
module builds that contract:

* ``input_ids`` [B, L]: per trajectory, the prompt tokens, then for each turn
  the policy's sampled tokens followed by the observation tokens the
  environment returned (the last turn's observation is left out unless asked
  for), padded with ``pad_id``;
* ``action_mask``, ``old_logprobs``, ``turn_ids`` [B, L-1], aligned with the
  causal targets ``input_ids[:, 1:]``: position i is the target at i+1, set
  where that token was sampled by the policy, with its stored behaviour
  log-probability (never recomputed from decoded text) and its turn;
* per-turn ``turn_rewards`` (sum of reward components), ``turn_mask`` and
  ``terminated`` [B, K] for the return/advantage estimators, whose per-turn
  advantages ``broadcast_turn_advantages(turn_adv, turn_ids, action_mask)``
  then aligns to the action tokens.

Host-side: the tensors are filled in NumPy, copied once into pinned host
memory and moved to ``device`` with one asynchronous copy each.  Overlong
streams raise instead of being truncated (training-pipeline.md:332-335).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Mapping, Optional, Sequence, Tuple, Union

import numpy as np
import torch
from torch import Tensor

from .trajectory import Trajectory

__all__ = ["PackedTrajectories", "pack_trajectories"]

ObservationTokens = Union[Mapping[str, Sequence[int]], Callable[[str], Sequence[int]]]


@dataclass(frozen=True)
class PackedTrajectories:
    input_ids: Tensor        # [B, L] int64
    attention_mask: Tensor   # [B, L] bool, True on real tokens
    action_mask: Tensor      # [B, L-1] bool, target input_ids[:, i+1] sampled by the policy
    old_logprobs: Tensor     # [B, L-1] behaviour log-prob of that target (0 elsewhere)
    turn_ids: Tensor         # [B, L-1] int64 turn of that target (0 elsewhere)
    turn_rewards: Tensor     # [B, K] float32 sum of each turn's reward components
    turn_mask: Tensor        # [B, K] bool, the turn exists
    terminated: Tensor       # [B, K] bool, the turn's transition is a true terminal
    lengths: Tensor          # [B] int64 real tokens per row
    policy_versions: Tuple[Tuple[str, ...], ...]  # per trajectory, per turn
    trajectory_ids: Tuple[str, ...]


def _resolver(observations: ObservationTokens) -> Callable[[str], Sequence[int]]:
    if callable(observations):
        return observations

    def look(ref: str) -> Sequence[int]:
        try:
            return observations[ref]
        except KeyError:
            raise KeyError(f"no observation tokens for observation_ref {ref!r}") from None
    return look


def pack_trajectories(
    trajectories: Sequence[Trajectory],
    prompt_token_ids: Sequence[Sequence[int]],
    observation_token_ids: ObservationTokens,
    *,
    pad_id: int = 0,
    max_length: Optional[int] = None,
    require_finished: bool = True,
    include_final_observation: bool = False,
    logprob_dtype: torch.dtype = torch.float32,
    device: Optional[Union[str, torch.device]] = None,
) -> PackedTrajectories:
    """Pack trajectories into the padded tensors of the training step.

    ``prompt_token_ids[b]`` are the tokens before trajectory b's first action
    (system and user turns; at least one, since the first sampled token is a
    target of the position before it).  ``observation_token_ids`` maps each
    transition's ``observation_ref`` to its tokens (a mapping or a callable).
    Every trajectory is validated first (``Trajectory.validate``).
    ``max_length`` fixes L (streams longer than it raise); by default L is the
    longest stream.  ``device`` (default: the host) receives every tensor.
    """

    B = len(trajectories)
    if len(prompt_token_ids) != B:
        raise ValueError(f"got {len(prompt_token_ids)} prompts for {B} trajectories")
    obs = _resolver(observation_token_ids)
    streams = []
    for b, traj in enumerate(trajectories):
        traj.validate(require_finished=require_finished)
        prompt = list(prompt_token_ids[b])
        if not prompt:
            raise ValueError("every trajectory needs at least one prompt token before its "
                             "first action")
        pieces = [(prompt, None)]
        last = len(traj.actions) - 1
        for k, (act, tr) in enumerate(zip(traj.actions, traj.transitions)):
            pieces.append((list(act.token_ids), act))
            if k < last or include_final_observation:
                pieces.append((list(obs(tr.observation_ref)), None))
        streams.append(pieces)

    lengths = np.array([sum(len(p) for p, _ in s) for s in streams], dtype=np.int64)
    L = int(lengths.max()) if B else 0
    if max_length is not None:
        over = np.nonzero(lengths > max_length)[0]
        if over.size:
            b = int(over[0])
            raise ValueError(f"trajectory {trajectories[b].trajectory_id!r} packs to "
                             f"{int(lengths[b])} tokens, more than max_length {max_length}")
        L = int(max_length)
    L = max(L, 1)
    K = max((len(t.actions) for t in trajectories), default=0)

    ids = np.full((B, L), pad_id, dtype=np.int64)
    att = np.zeros((B, L), dtype=bool)
    amask = np.zeros((B, L - 1), dtype=bool)
    old = np.zeros((B, L - 1), dtype=np.float64)
    turn = np.zeros((B, L - 1), dtype=np.int64)
    rew = np.zeros((B, K), dtype=np.float32)
    tmask = np.zeros((B, K), dtype=bool)
    term = np.zeros((B, K), dtype=bool)
    for b, pieces in enumerate(streams):
        pos = 0
        for toks, act in pieces:
            n = len(toks)
            ids[b, pos:pos + n] = toks
            if act is not None:
                # token at stream position p is the target of position p - 1
                amask[b, pos - 1:pos - 1 + n] = True
                old[b, pos - 1:pos - 1 + n] = act.old_logprobs
                turn[b, pos - 1:pos - 1 + n] = act.turn
            pos += n
        att[b, :pos] = True
        for k, tr in enumerate(trajectories[b].transitions):
            rew[b, k] = sum(tr.reward_components.values())
            tmask[b, k] = True
            term[b, k] = tr.terminated

    def move(a: np.ndarray, dtype: Optional[torch.dtype] = None) -> Tensor:
        t = torch.from_numpy(a)
        if dtype is not None:
            t = t.to(dtype)
        if device is None or torch.device(device).type == "cpu":
            return t
        return t.pin_memory().to(device, non_blocking=True)

    out = PackedTrajectories(
        input_ids=move(ids),
        attention_mask=move(att),
        action_mask=move(amask),
        old_logprobs=move(old, logprob_dtype),
        turn_ids=move(turn),
        turn_rewards=move(rew),
        turn_mask=move(tmask),
        terminated=move(term),
        lengths=move(lengths),
        policy_versions=tuple(tuple(a.policy_version for a in t.actions) for t in trajectories),
        trajectory_ids=tuple(t.trajectory_id for t in trajectories),
    )
    if device is not None and torch.device(device).type != "cpu":
        # the pinned staging buffers must outlive the asynchronous copies
        torch.cuda.current_stream(torch.device(device)).synchronize()
    return out
