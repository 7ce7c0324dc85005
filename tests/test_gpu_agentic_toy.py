"""End-to-end GRPO training through the HIP path: the reference's integration
harness (examples/agentic_rl_toy.py:65-162) restated on this package.

A table policy of logits [task, turn, action] must learn four 3-step action
paths from group-relative terminal rewards.  Each step: sample a group of
paths per task from a frozen snapshot (on the CPU, with the harness's seeded
generator), verify them, standardize rewards within each group
(group_standardized_advantages), broadcast each path's advantage to its action
tokens, recompute log-probs (gather_token_logprobs), take the clipped loss
(clipped_policy_loss) and an Adam step.  The harness's pass criterion is
greedy accuracy 1.0 after 150 steps (seed 7, group 32, lr 0.05); the same run
through fused_policy_loss must pass too.
"""

from __future__ import annotations

import pytest
import torch

from rosellm_amd import roserlhf as R

pytestmark = pytest.mark.gpu

# The task table of the harness (examples/agentic_rl_toy.py:31-39): the
# rewarded action path of each task.
PATHS = torch.tensor([[0, 0, 1], [0, 1, 0], [1, 0, 1], [1, 1, 0]], dtype=torch.long)


def _train(device, fused: bool, steps=150, group=32, lr=0.05, seed=7):
    torch.manual_seed(seed)
    gen = torch.Generator().manual_seed(seed + 1)
    n_tasks, horizon = PATHS.shape
    table = torch.nn.Parameter(torch.zeros(n_tasks, horizon, 2, device=device))
    opt = torch.optim.Adam([table], lr=lr)
    tasks = torch.arange(n_tasks).repeat_interleave(group)
    tasks_d = tasks.to(device)
    for _ in range(steps):
        with torch.no_grad():
            probs = table.detach().cpu()[tasks].softmax(dim=-1)
            acts = torch.multinomial(probs.reshape(-1, 2), 1, generator=gen).reshape(-1, horizon)
            rewards = (acts == PATHS[tasks]).all(dim=-1).float()
            acts_d = acts.to(device)
            old = R.gather_token_logprobs(table[tasks_d], acts_d)
        adv = R.group_standardized_advantages(rewards.to(device).reshape(-1, group)).reshape(-1)
        tok_adv = adv[:, None].expand(-1, horizon)
        mask = torch.ones(tasks.numel(), horizon, dtype=torch.bool, device=device)
        if fused:
            out = R.fused_policy_loss(table[tasks_d], acts_d, old, tok_adv, mask, clip_low=0.2)
        else:
            cur = R.gather_token_logprobs(table[tasks_d], acts_d)
            out = R.clipped_policy_loss(cur, old, tok_adv, mask, clip_low=0.2)
        opt.zero_grad(set_to_none=True)
        out.loss.backward()
        opt.step()
    greedy = table.detach().cpu().argmax(dim=-1)
    return (greedy == PATHS).all(dim=-1).float().mean().item()


@pytest.mark.parametrize("fused", [False, True])
def test_agentic_toy_reaches_full_accuracy(device, fused):
    print(f"[agentic-toy] fused={fused}", flush=True)
    assert _train(device, fused) == 1.0
