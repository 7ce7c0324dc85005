"""Trajectory records (rosellm/roserlhf/trajectory.py) and their packing into
the training step's tensors, on the CPU.

The record tests restate the reference's tests/test_roserlhf_trajectory.py
cases (same inputs, same expected messages).  Packing is pinned by a
hand-built sequence (docs/agentic-rl/training-pipeline.md:324-326: logits at
position i score input_ids[i+1]), by an independent per-token restatement
on random trajectories, and by the docs' invariant that padding leaves the
globally normalized loss unchanged (mathematical-foundations.md:654-655).
"""

from __future__ import annotations

import random

import pytest
import torch

from oracle import roserlhf_oracle as o
from rosellm_amd.roserlhf import pack_trajectories
from rosellm_amd.roserlhf.trajectory import PolicyAction, Trajectory, TransitionRecord


def make_action(turn, policy="policy-1", tokens=(10, 11), lps=(-0.2, -0.5)):
    return PolicyAction(turn=turn, token_ids=list(tokens), old_logprobs=list(lps),
                        policy_version=policy, text="search",
                        parsed_action={"tool": "search", "query": "evidence"})


def make_transition(turn, *, terminal=False, reward=None):
    r = float(terminal) if reward is None else reward
    return TransitionRecord(turn=turn, observation_ref=f"sha256:observation-{turn}",
                            reward_components={"success": r}, terminated=terminal)


# --- the reference's record tests, restated ---------------------------------


def test_policy_action_requires_exact_logprob_per_token():
    with pytest.raises(ValueError, match="every sampled token"):
        PolicyAction(turn=0, token_ids=[1, 2], old_logprobs=[-0.1], policy_version="v1", text="x")


def test_trajectory_orders_turns_and_tracks_mixed_policy_versions():
    t = Trajectory(trajectory_id="traj-1", task_id="task-1", environment_version="env-3",
                   tokenizer_hash="sha256:tokenizer")
    t.append(make_action(0, "v1"), make_transition(0))
    t.append(make_action(1, "v2"), make_transition(1, terminal=True))
    t.validate()
    assert t.is_finished
    assert t.behavior_policy_versions == ["v1", "v2"]


def test_trajectory_rejects_append_after_terminal():
    t = Trajectory("t", "q", "env", "tok")
    t.append(make_action(0), make_transition(0, terminal=True))
    with pytest.raises(ValueError, match="finished"):
        t.append(make_action(1), make_transition(1))


def test_trajectory_can_validate_partial_rollout_explicitly():
    t = Trajectory("t", "q", "env", "tok")
    t.append(make_action(0), make_transition(0))
    t.validate(require_finished=False)
    with pytest.raises(ValueError, match="incomplete"):
        t.validate()


# --- the remaining validation rules of the record types ----------------------


@pytest.mark.parametrize("kw,msg", [
    (dict(turn=-1), "turn must be non-negative"),
    (dict(policy_version=""), "policy_version is required"),
    (dict(token_ids=[], old_logprobs=[]), "at least one token"),
    (dict(token_ids=[3, -1], old_logprobs=[0.0, 0.0]), "non-negative"),
])
def test_policy_action_rules(kw, msg):
    base = dict(turn=0, token_ids=[1], old_logprobs=[-1.0], policy_version="v", text="")
    with pytest.raises(ValueError, match=msg):
        PolicyAction(**{**base, **kw})


def test_transition_and_trajectory_rules():
    with pytest.raises(ValueError, match="observation_ref is required"):
        TransitionRecord(turn=0, observation_ref="")
    with pytest.raises(ValueError, match="both terminated and truncated"):
        TransitionRecord(turn=0, observation_ref="o", terminated=True, truncated=True)
    t = Trajectory("t", "q", "env", "tok")
    with pytest.raises(ValueError, match="expected turn 0"):
        t.append(make_action(1), make_transition(1))
    t.actions.append(make_action(0))
    with pytest.raises(ValueError, match="one transition"):
        t.validate(require_finished=False)
    t2 = Trajectory("t", "q", "env", "tok", actions=[make_action(0), make_action(1)],
                    transitions=[make_transition(0, terminal=True), make_transition(1)])
    with pytest.raises(ValueError, match="no events may follow"):
        t2.validate(require_finished=False)
    with pytest.raises(ValueError, match="trajectory_id and task_id"):
        Trajectory("", "q", "env", "tok").validate(require_finished=False)
    with pytest.raises(ValueError, match="environment_version and tokenizer_hash"):
        Trajectory("t", "q", "", "tok").validate(require_finished=False)


# --- packing -----------------------------------------------------------------


def test_pack_hand_built_sequence():
    t = Trajectory("traj", "task", "env", "tok")
    t.append(make_action(0, "v1", (10, 11), (-0.2, -0.5)), make_transition(0, reward=0.25))
    t.append(make_action(1, "v2", (12,), (-0.7,)), make_transition(1, terminal=True))
    obs = {"sha256:observation-0": [20, 21, 22], "sha256:observation-1": [99]}
    p = pack_trajectories([t], [[1, 2, 3]], obs)
    # stream: prompt 1 2 3 | action0 10 11 | obs0 20 21 22 | action1 12
    assert p.input_ids.tolist() == [[1, 2, 3, 10, 11, 20, 21, 22, 12]]
    # targets input_ids[:, 1:] = 2 3 10 11 20 21 22 12
    assert p.action_mask.tolist() == [[False, False, True, True, False, False, False, True]]
    assert p.old_logprobs.tolist() == [[0, 0, torch.tensor(-0.2).item(), torch.tensor(-0.5).item(),
                                        0, 0, 0, torch.tensor(-0.7).item()]]
    assert p.turn_ids.tolist() == [[0, 0, 0, 0, 0, 0, 0, 1]]
    assert p.turn_rewards.tolist() == [[0.25, 1.0]]
    assert p.terminated.tolist() == [[False, True]]
    assert p.policy_versions == (("v1", "v2"),) and p.lengths.tolist() == [9]
    q = pack_trajectories([t], [[1, 2, 3]], obs, include_final_observation=True, pad_id=-1,
                          max_length=12)
    assert q.input_ids.tolist() == [[1, 2, 3, 10, 11, 20, 21, 22, 12, 99, -1, -1]]
    assert q.attention_mask.sum().item() == 10


def _random_batch(seed, B=6):
    rng = random.Random(seed)
    trajs, prompts, obs = [], [], {}
    for b in range(B):
        t = Trajectory(f"t{b}", f"task{b // 2}", "env", "tok")
        K = rng.randint(1, 4)
        for k in range(K):
            n = rng.randint(1, 5)
            toks = [rng.randrange(100, 200) for _ in range(n)]
            lps = [-rng.random() * 3 for _ in range(n)]
            ref = f"obs-{b}-{k}"
            obs[ref] = [rng.randrange(200, 300) for _ in range(rng.randint(0, 4))]
            t.append(PolicyAction(k, toks, lps, f"v{rng.randint(0, 1)}", ""),
                     TransitionRecord(k, ref, {"r": rng.random(), "bonus": 1.0},
                                      terminated=(k == K - 1)))
        trajs.append(t)
        prompts.append([rng.randrange(1, 100) for _ in range(rng.randint(1, 6))])
    return trajs, prompts, obs


def _restated(trajs, prompts, obs):
    """Independent per-token restatement: one (token, sampled?, logp, turn)
    record per stream position, then the causal shift."""

    rows = []
    for t, prompt in zip(trajs, prompts):
        recs = [(tok, False, 0.0, 0) for tok in prompt]
        for k, a in enumerate(t.actions):
            recs += [(tok, True, lp, a.turn) for tok, lp in zip(a.token_ids, a.old_logprobs)]
            if k < len(t.actions) - 1:
                recs += [(tok, False, 0.0, 0) for tok in obs[t.transitions[k].observation_ref]]
        rows.append(recs)
    return rows


def test_pack_matches_restatement_on_random_trajectories():
    trajs, prompts, obs = _random_batch(3)
    p = pack_trajectories(trajs, prompts, obs.__getitem__, pad_id=7, logprob_dtype=torch.float64)
    L = p.input_ids.shape[1]
    for b, recs in enumerate(_restated(trajs, prompts, obs)):
        n = len(recs)
        assert p.lengths[b].item() == n
        assert p.input_ids[b, :n].tolist() == [r[0] for r in recs]
        assert (p.input_ids[b, n:] == 7).all() and (p.attention_mask[b].sum() == n)
        shifted = recs[1:] + [(7, False, 0.0, 0)] * (L - n)
        assert p.action_mask[b].tolist() == [r[1] for r in shifted]
        assert p.old_logprobs[b].tolist() == [r[2] for r in shifted]  # bit-exact in float64
        assert p.turn_ids[b].tolist() == [r[3] for r in shifted]
        K = len(trajs[b].actions)
        assert p.turn_mask[b].sum().item() == K
        assert p.turn_rewards[b, :K].tolist() == pytest.approx(
            [sum(tr.reward_components.values()) for tr in trajs[b].transitions], rel=1e-7)


def test_padding_leaves_globally_normalized_loss_unchanged():
    """Same tokens, more padding: the action positions, their stored
    log-probs and turns move nowhere, so the globally token-normalized loss of
    the same per-token log-probs is unchanged (padded positions hold junk)."""

    trajs, prompts, obs = _random_batch(5)
    a = pack_trajectories(trajs, prompts, obs)
    b = pack_trajectories(trajs, prompts, obs, max_length=a.input_ids.shape[1] + 9, pad_id=3)
    n = a.action_mask.shape[1]
    assert torch.equal(a.action_mask, b.action_mask[:, :n]) and not b.action_mask[:, n:].any()
    turn_adv = torch.linspace(-1, 1, 4).expand(len(trajs), 4).contiguous()
    noise = 0.1 * torch.randn(a.old_logprobs.shape, generator=torch.Generator().manual_seed(1))
    cur_a = a.old_logprobs + noise
    cur_b = torch.full(b.old_logprobs.shape, 123.0)
    cur_b[:, :n] = cur_a

    def loss(p, cur):
        adv = o.turn_broadcast(turn_adv, p.turn_ids, p.action_mask)
        return o.ppo_clip(cur, p.old_logprobs, adv, p.action_mask, clip_low=0.2)["loss"].item()

    la, lb = loss(a, cur_a), loss(b, cur_b)
    assert abs(la - lb) <= 1e-6 * abs(la)


def test_pack_errors():
    trajs, prompts, obs = _random_batch(9, B=2)
    with pytest.raises(ValueError, match="prompts for 2 trajectories"):
        pack_trajectories(trajs, prompts[:1], obs)
    with pytest.raises(ValueError, match="at least one prompt token"):
        pack_trajectories(trajs, [[], [1]], obs)
    with pytest.raises(ValueError, match="more than max_length"):
        pack_trajectories(trajs, prompts, obs, max_length=3)
    with pytest.raises(KeyError, match="no observation tokens"):
        pack_trajectories(trajs, prompts, {})
    open_t = Trajectory("t", "q", "env", "tok")
    open_t.append(make_action(0), make_transition(0))
    with pytest.raises(ValueError, match="incomplete"):
        pack_trajectories([open_t], [[1]], {"sha256:observation-0": [5]})
    p = pack_trajectories([open_t], [[1]], {}, require_finished=False)
    assert p.input_ids.tolist() == [[1, 10, 11]] and not p.terminated.any()
