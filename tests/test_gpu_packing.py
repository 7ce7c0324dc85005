"""Trajectory records -> packed tensors on the GPU -> GRPO step on the HIP
path, against the CPU oracle on the same packed tensors (MI355X).

The causal alignment is the reference's (training-pipeline.md:340-348):
logits[:, :-1] score input_ids[:, 1:], action_mask / old_logprobs / turn_ids
sit on the target positions, and broadcast_turn_advantages aligns per-turn
advantages to the action tokens.  Bars as in test_gpu_parity: bit-exact
advantages and masks, bf16 loss within 2e-3, dlogits rows within 2e-3
norm-wise of the correctly rounded exact rows.
"""

from __future__ import annotations

import random

import pytest
import torch

from oracle import roserlhf_oracle as o
from rosellm_amd import roserlhf as R
from rosellm_amd.roserlhf.trajectory import PolicyAction, Trajectory, TransitionRecord

from test_gpu_parity import _rownorm16

pytestmark = pytest.mark.gpu


def _batch(seed, groups=3, G=4, V=4096):
    rng = random.Random(seed)
    trajs, prompts, obs = [], [], {}
    for b in range(groups * G):
        t = Trajectory(f"t{b}", f"task{b // G}", "env", "tok")
        K = rng.randint(1, 4)
        for k in range(K):
            n = rng.randint(1, 12)
            toks = [rng.randrange(V) for _ in range(n)]
            lps = [-3.0 * rng.random() for _ in range(n)]
            ref = f"o{b}.{k}"
            obs[ref] = [rng.randrange(V) for _ in range(rng.randint(0, 6))]
            last = k == K - 1
            t.append(PolicyAction(k, toks, lps, "v1", ""),
                     TransitionRecord(k, ref, {"success": float(last and rng.random() < 0.5)},
                                      terminated=last))
        trajs.append(t)
        prompts.append([rng.randrange(V) for _ in range(rng.randint(1, 8))])
    return trajs, prompts, obs


def test_packed_grpo_step_matches_oracle(device):
    G, V = 4, 4096
    trajs, prompts, obs = _batch(7, G=G, V=V)
    p = R.pack_trajectories(trajs, prompts, obs, device=device)
    pc = R.pack_trajectories(trajs, prompts, obs)
    for name in ("input_ids", "action_mask", "old_logprobs", "turn_ids", "turn_rewards"):
        assert torch.equal(getattr(p, name).cpu(), getattr(pc, name)), name
    B, L = p.input_ids.shape
    K = p.turn_mask.shape[1]
    # GRPO: terminal reward per trajectory, group-standardized, one value per turn
    reward = (p.turn_rewards * p.turn_mask).sum(dim=1)
    seq_adv = R.group_standardized_advantages(reward.view(-1, G)).reshape(-1)
    turn_adv = seq_adv[:, None].expand(B, K).contiguous()
    tok_adv = R.broadcast_turn_advantages(turn_adv, p.turn_ids, p.action_mask)
    seq_o = o.group_standardize(reward.cpu().view(-1, G)).reshape(-1)
    tok_o = o.turn_broadcast(seq_o[:, None].expand(B, K).contiguous(), pc.turn_ids,
                             pc.action_mask)
    assert torch.equal(tok_adv.cpu(), tok_o), "token advantages differ"

    g = torch.Generator().manual_seed(11)
    x = (torch.randn(B, L, V, generator=g) * 3.0).to(torch.bfloat16)
    xd = x.to(device).requires_grad_()
    out = R.fused_policy_loss(xd[:, :-1], p.input_ids[:, 1:], p.old_logprobs, tok_adv,
                              p.action_mask, clip_low=0.2, clip_high=0.28)
    out.loss.backward()
    ref, _lp, dl = o.policy_step("ppo", x[:, :-1], pc.input_ids[:, 1:], pc.old_logprobs, tok_o,
                                 pc.action_mask, exact=True, clip_low=0.2, clip_high=0.28)
    assert abs(out.loss.item() - ref["loss"].item()) <= 2e-3 * max(abs(ref["loss"].item()), 1e-3)
    assert (xd.grad[:, -1] == 0).all()
    _rownorm16(xd.grad[:, :-1], dl, 2e-3, "packed dlogits")
