#!/usr/bin/env python3
"""Throughput of the RoseRLHF GRPO training-step hot path on one MI355X.

Workload (config 2, the headline): 32 prompts x group 8 = 256 sequences x 1024
tokens, vocabulary 151936, bf16 logits ~ N(0, 3) with 5% of rows given one
dominant logit (+15).  Actions are sampled from softmax(logits) (Gumbel-max,
exact), old_logprobs = logprobs + N(0, 0.1), rewards uniform {0, 1} per
sequence, response lengths uniform [64, 1024] (mask = t < length), clip
eps_low 0.2 / eps_high 0.28, token-mean loss.

One timed step = group-standardized advantages (advantages.py:236-258)
broadcast to tokens (examples/agentic_rl_toy.py:104-106) -> log-probs of the
actions (losses.py:14-38) -> clipped_policy_loss (losses.py:426-486) ->
backward to bf16 dlogits.  ``--path fused`` (default) runs it through
``fused_policy_loss``, one read of the logits and one write of dlogits;
``--path composed`` runs ``gather_token_logprobs`` then
``clipped_policy_loss`` and autograd (two reads, one write).  Inputs are
resident in HBM before the timed region.

``--config c5`` is the fused LM-head step: hidden [256x1024, 1024] bf16 and
an LM-head weight [151936, 1024] bf16 -> log-probs -> clipped objective ->
d hidden and d weight, through ``fused_linear_policy_loss`` (``--path
composed``: F.linear, gather_token_logprobs, clipped_policy_loss, autograd);
its roofline is MFMA-bound (3 x 2*N*H*V flops per step).

``--config sample`` is the rollout side: one decode step of 256 rows x
151936 bf16 logits -> next token + behaviour log-probs
(``rosellm_amd.roseinfer.sample_next_token_batch``, roseinfer/engine.py:
1103-1171 defaults T = 1, top_k = 0, top_p = 1; a top-k/top-p variant beside it).

``--config sft`` is the supervised next-token cross-entropy of the model
forwards (rosetrainer/model.py:643-649) on config 2's logits, labels = the
sampled tokens: ``rosellm_amd.rosetrainer.causal_lm_loss`` (the same
single-pass row kernel, objective NLL) -> backward to bf16 dlogits.

Prints one JSON line (rank 0): value = tokens/s over all B*T positions, plus
``roofline`` for the dominant kernel (HIP events around its entry point over
the timed steps; algorithmic bytes N*(V*(2+2) + 21)) and ``cpu_baseline``, the
oracle's PyTorch-CPU composition timed on a bounded sub-batch of the same
tensors.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "tokens/sec for logprob+GRPO loss fwd+bwd @151936 vocab; % of HBM roofline"
HBM_PEAK_GBS = 8000.0
SIDE_BYTES = 21  # per token: 8 target + 4 old logp + 4 advantage + 1 mask + 4 logp out

CONFIGS = {
    # c2 is the headline workload; the others are run on request (--config).
    "c2": dict(prompts=32, group=8, T=1024, V=151936, dtype="bfloat16", sigma=3.0, hot=0.05,
               noise=0.1, lengths=(64, 1024), rewards="uniform01", objective="clipped",
               kw=dict(clip_low=0.2, clip_high=0.28),
               workload="C2: GRPO token-level PPO-clip fwd+bwd, 256x1024 tokens, V=151936 bf16"),
    "c1": dict(prompts=8, group=4, T=128, V=50257, dtype="float32", sigma=2.0, hot=0.0,
               noise=0.05, lengths=(16, 128), rewards="bernoulli0.3", objective="clipped",
               kw=dict(clip_low=0.2, clip_high=None),
               workload="C1: GRPO token-level PPO-clip fwd+bwd, 32x128 tokens, V=50257 fp32"),
    "c3": dict(prompts=32, group=8, T=1024, V=151936, dtype="bfloat16", sigma=3.0, hot=0.05,
               noise=0.1, lengths=(64, 1024), rewards="bernoulli0.5", objective="gspo",
               kw=dict(clip_low=3e-4, clip_high=4e-4),
               workload="C3: GSPO sequence-level objective fwd+bwd, 256x1024 tokens, V=151936 bf16"),
    "c4": dict(prompts=64, group=1, T=8192, V=151936, dtype="bfloat16", sigma=3.0, hot=0.05,
               noise=0.1, lengths=(1024, 8192), rewards="terminal_normal", objective="sapo",
               kw=dict(tau_positive=1.0, tau_negative=1.0),
               workload="C4: GAE(gamma 1, lambda 0.95) + masked whitening + SAPO fwd+bwd, "
                        "64x8192 tokens, V=151936 bf16, dlogits in place"),
    "c5": dict(prompts=32, group=8, T=1024, V=151936, H=1024, dtype="bfloat16", sigma=1.0,
               w_sigma=0.02, hot=0.0, noise=0.1, lengths=(64, 1024), rewards="uniform01",
               objective="clipped", kw=dict(clip_low=0.2, clip_high=0.28), lm_head=True,
               workload="C5: fused LM-head + logprob + GRPO PPO-clip fwd+bwd to dhidden and dW, "
                        "256x1024 tokens, hidden 1024, V=151936 bf16"),
}
CONFIGS["sft"] = dict(CONFIGS["c2"], objective="nll", kw={}, sft=True,
                      workload="SFT: next-token cross-entropy fwd+bwd (rosetrainer/model.py:"
                               "643-649), 256x1024 tokens, V=151936 bf16")
SFT_SIDE_BYTES = 12  # per row: 8 label + 4 logp out
LM_HEAD_ROW_BLOCK = 16384
MFMA_BF16_PEAK_TFLOPS = 2500.0
def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=None,
                   help="timed steps (default 10; 200 for c1 and the sampler, whose steps "
                        "are under 1 ms)")
    p.add_argument("--warmup", type=int, default=None,
                   help="untimed steps first (default 2; 20 for c1 and the sampler, whose "
                        "host-bound steps settle over more calls)")
    p.add_argument("--config", choices=sorted(CONFIGS) + ["sample"], default="c2")
    p.add_argument("--path", choices=["fused", "composed"], default="fused")
    p.add_argument("--objective", choices=["gspo", "gspo_token"], default=None,
                   help="config c3 only: GSPO (default) or GSPO-token")
    p.add_argument("--cpu-sample-seqs", type=int, default=2,
                   help="sequences of the batch timed on the CPU oracle")
    p.add_argument("--cpu-runs", type=int, default=3)
    p.add_argument("--skip-cpu", action="store_true")
    p.add_argument("--no-variants", action="store_true",
                   help="do not also time the skip_masked_rows variant of the fused path")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="also launch one device copy of known size (HBM counter calibration)")
    p.add_argument("--seed", type=int, default=1234)
    return p.parse_args()


def make_inputs(cfg, device, seed):
    """Synthetic config tensors on the GPU.  One generator seed per tensor:
    seed + tensor index."""

    import torch

    B = cfg["prompts"] * cfg["group"]
    T, V = cfg["T"], cfg["V"]
    dtype = getattr(torch, cfg["dtype"])
    gens = [torch.Generator(device=device).manual_seed(seed + i) for i in range(10)]
    hidden = weight = logits = None
    if cfg.get("lm_head"):
        # Config 5: hidden ~ N(0, 1), LM-head weight ~ N(0, w_sigma); the
        # logits exist only one row chunk at a time, as products of the two.
        H = cfg["H"]
        hidden = torch.randn(B, T, H, dtype=dtype, device=device, generator=gens[8])
        hidden.mul_(cfg["sigma"])
        weight = torch.randn(V, H, dtype=dtype, device=device, generator=gens[9])
        weight.mul_(cfg["w_sigma"])
        h2 = hidden.view(-1, H)
        row_logits = lambda r0, r1: torch.mm(h2[r0:r1], weight.t())
    else:
        logits = torch.randn(B, T, V, dtype=dtype, device=device, generator=gens[0])
        logits.mul_(cfg["sigma"])
        flat = logits.view(-1, V)
        if cfg["hot"] > 0:
            hot_rows = torch.nonzero(torch.rand(B * T, device=device, generator=gens[1])
                                     < cfg["hot"])
            hot_rows = hot_rows.reshape(-1)
            hot_cols = torch.randint(0, V, (hot_rows.numel(),), device=device,
                                     generator=gens[2])
            flat[hot_rows, hot_cols] = (flat[hot_rows, hot_cols].float() + 15.0).to(dtype)
        row_logits = lambda r0, r1: flat[r0:r1]
    # Actions ~ softmax(logits) by Gumbel-max; reference log-probs by
    # log_softmax in float32, chunked so no [N, V] float32 tensor is built.
    actions = torch.empty(B * T, dtype=torch.int64, device=device)
    logp = torch.empty(B * T, dtype=torch.float32, device=device)
    chunk = max(1, (1 << 30) // (V * 4))
    for r0 in range(0, B * T, chunk):
        xf = row_logits(r0, min(B * T, r0 + chunk)).float()
        u = torch.rand(xf.shape, device=device, generator=gens[3]).clamp_(min=1e-20)
        a = torch.argmax(xf - torch.log(-torch.log(u)), dim=-1)
        actions[r0:r0 + chunk] = a
        logp[r0:r0 + chunk] = torch.log_softmax(xf, dim=-1).gather(1, a[:, None]).squeeze(1)
        del xf, u
    actions = actions.view(B, T)
    old = (logp + cfg["noise"] * torch.randn(B * T, device=device, generator=gens[4])).view(B, T)
    lo, hi = cfg["lengths"]
    lengths = torch.randint(lo, hi + 1, (B,), device=device, generator=gens[6])
    mask = torch.arange(T, device=device)[None, :] < lengths[:, None]
    shape = (cfg["prompts"], cfg["group"])
    values = None
    if cfg["rewards"] == "uniform01":
        rewards = torch.randint(0, 2, shape, device=device, generator=gens[5]).float()
    elif cfg["rewards"].startswith("bernoulli"):
        p = float(cfg["rewards"][len("bernoulli"):])
        rewards = (torch.rand(shape, device=device, generator=gens[5]) < p).float()
    else:  # per-token rewards: 0 except a terminal N(0, 1) at t = length - 1
        rewards = torch.zeros(B, T, device=device)
        rewards[torch.arange(B, device=device), lengths - 1] = torch.randn(
            B, device=device, generator=gens[5])
        values = 0.5 * torch.randn(B, T, device=device, generator=gens[7])
    return dict(logits=logits, hidden=hidden, weight=weight, actions=actions, old=old,
                rewards=rewards, values=values, mask=mask, B=B, T=T, V=V)


def _watch(lp, probe):
    if probe is not None:
        lp.register_hook(lambda g: probe.__setitem__("active", int((g != 0).sum().item())))


def make_step(inp, cfg, path, objective, skip_masked=False, probe=None):
    """One timed step of the config's training-step hot path.  With ``probe``
    (a dict; composed path only, never in a timed step) the step also records
    how many token rows receive a non-zero d loss / d logp: the backward
    kernel reads the logits of those rows only."""

    from rosellm_amd import roserlhf as R

    actions, old, rewards, mask = inp["actions"], inp["old"], inp["rewards"], inp["mask"]
    B, T = inp["B"], inp["T"]
    kw = cfg["kw"]

    if cfg.get("lm_head"):
        # Config 5: hidden -> LM head -> log-probs -> clipped objective ->
        # d hidden, d weight.  "fused" never holds more than one row block of
        # logits; "composed" is the reference's chain (F.linear, then
        # gather_token_logprobs and clipped_policy_loss, autograd through all).
        import torch.nn.functional as F

        hidden = inp["hidden"].requires_grad_()
        weight = inp["weight"].requires_grad_()

        def step():
            hidden.grad = None
            weight.grad = None
            a = R.group_standardized_advantages(rewards).reshape(-1)[:, None].expand(B, T)
            if path == "fused":
                out = R.fused_linear_policy_loss(hidden, weight, actions, old, a, mask,
                                                 row_block=LM_HEAD_ROW_BLOCK, **kw)
            else:
                lp = R.gather_token_logprobs(F.linear(hidden, weight), actions)
                _watch(lp, probe)
                out = R.clipped_policy_loss(lp, old, a, mask, **kw)
            out.loss.backward()
            return out
        return step

    logits = inp["logits"].requires_grad_()

    if cfg.get("sft"):
        # SFT loss of the model forwards: position t scores label t+1.
        from types import SimpleNamespace

        from rosellm_amd import rosetrainer as RT

        def step():
            logits.grad = None
            loss = RT.causal_lm_loss(logits, actions)
            loss.backward()
            return SimpleNamespace(loss=loss)
        return step

    if objective == "sapo":
        # Config 4: GAE over the valid tokens, whitened, then SAPO.  dlogits
        # overwrite the logits (logits + dlogits would need 318.6 GB), so each
        # step after the first runs on the previous step's dlogits: the same
        # work on different values.
        def step():
            logits.grad = None
            adv, _ = R.generalized_advantage_estimation(rewards, inp["values"], gamma=1.0,
                                                        gae_lambda=0.95, valid_mask=mask)
            adv = R.masked_whiten(adv, mask)
            out = R.fused_policy_loss(logits, actions, old, adv, mask, objective="sapo",
                                      inplace=True, **kw)
            out.loss.backward()
            return out
        return step

    def advantages():
        seq = R.group_standardized_advantages(rewards).reshape(-1)
        return seq if objective == "gspo" else seq[:, None].expand(B, T)

    if path == "fused":
        def step():
            logits.grad = None
            out = R.fused_policy_loss(logits, actions, old, advantages(), mask,
                                      objective=objective, skip_masked_rows=skip_masked, **kw)
            out.loss.backward()
            return out
    else:
        fn = {"clipped": R.clipped_policy_loss, "gspo": R.gspo_policy_loss,
              "gspo_token": R.gspo_token_policy_loss}[objective]

        def step():
            logits.grad = None
            lp = R.gather_token_logprobs(logits, actions)
            _watch(lp, probe)
            out = fn(lp, old, advantages(), mask, **kw)
            out.loss.backward()
            return out
    return step


def cpu_baseline(inp, cfg, n_seq, runs):
    """The oracle's PyTorch-CPU composition (log_softmax -> gather -> clip ->
    autograd), op for op the reference's, timed on the first n_seq sequences."""

    import torch

    from oracle import roserlhf_oracle as o

    T = inp["T"]
    if cfg.get("lm_head"):
        return cpu_baseline_lm_head(inp, cfg, n_seq, runs)
    x = inp["logits"].detach()[:n_seq].cpu()
    t = inp["actions"][:n_seq].cpu()
    if cfg.get("sft"):
        return cpu_baseline_sft(x, t, inp, n_seq, runs)
    old = inp["old"][:n_seq].cpu()
    mask = inp["mask"][:n_seq].cpu()
    objective = cfg["objective"]
    if objective == "sapo":
        adv, _ = o.gae(inp["rewards"][:n_seq].cpu(), inp["values"][:n_seq].cpu(), gamma=1.0,
                       gae_lambda=0.95, valid_mask=mask)
        adv = o.masked_whiten(adv, mask)
    else:
        seq_adv = o.group_standardize(inp["rewards"].cpu()).reshape(-1)[:n_seq]
        adv = seq_adv if objective == "gspo" else seq_adv[:, None].expand(n_seq, T)
    kind = {"clipped": "ppo"}.get(objective, objective)
    threads = torch.get_num_threads()
    times = []
    for i in range(runs + 1):
        t0 = time.perf_counter()
        o.policy_step(kind, x, t, old, adv, mask, **cfg["kw"])
        dt = time.perf_counter() - t0
        if i > 0:
            times.append(dt)
        log(f"[bench] cpu oracle run {i}: {dt:.2f} s")
    med = statistics.median(times)
    return {
        "value": round(n_seq * T / med, 1),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"first {n_seq} of {inp['B']} sequences ({n_seq * T} token rows, same "
                   f"tensors), oracle log_softmax->gather->{objective}->autograd on the fp32 "
                   f"upcast, "
                   f"median of {runs} runs after 1 warm-up, torch threads={threads}, "
                   f"os.cpu_count()={os.cpu_count()}"),
    }


def cpu_baseline_sft(x, t, inp, n_seq, runs):
    """SFT loss on the CPU: the oracle's shift -> log_softmax -> gather ->
    mean -> autograd on the float32 upcast of the first n_seq sequences."""

    import torch

    from oracle import roserlhf_oracle as o

    T = inp["T"]
    threads = torch.get_num_threads()
    times = []
    for i in range(runs + 1):
        t0 = time.perf_counter()
        o.sft_step(x, t, causal=True)
        dt = time.perf_counter() - t0
        if i > 0:
            times.append(dt)
        log(f"[bench] cpu oracle run {i}: {dt:.2f} s")
    med = statistics.median(times)
    return {
        "value": round(n_seq * T / med, 1),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"first {n_seq} of {inp['B']} sequences ({n_seq * T} token rows, same "
                   f"tensors), oracle shift->log_softmax->gather->mean->autograd on the fp32 "
                   f"upcast, median of {runs} runs after 1 warm-up, torch threads={threads}, "
                   f"os.cpu_count()={os.cpu_count()}"),
    }


def cpu_baseline_lm_head(inp, cfg, n_seq, runs):
    """Config 5 on the CPU: the reference chain (hidden @ W.T, log_softmax,
    gather, clipped objective, autograd back through the linear map) in
    float32 on the first n_seq sequences."""

    import torch

    from oracle import roserlhf_oracle as o

    T = inp["T"]
    h = inp["hidden"].detach()[:n_seq].cpu().float()
    w = inp["weight"].detach().cpu().float()
    t = inp["actions"][:n_seq].cpu()
    old = inp["old"][:n_seq].cpu()
    mask = inp["mask"][:n_seq].cpu()
    seq_adv = o.group_standardize(inp["rewards"].cpu()).reshape(-1)[:n_seq]
    adv = seq_adv[:, None].expand(n_seq, T)
    threads = torch.get_num_threads()
    times = []
    for i in range(runs + 1):
        t0 = time.perf_counter()
        x = h @ w.t()
        o.lm_head_step("ppo", h, w, x, t, old, adv, mask, **cfg["kw"])
        dt = time.perf_counter() - t0
        del x
        if i > 0:
            times.append(dt)
        log(f"[bench] cpu oracle run {i}: {dt:.2f} s")
    med = statistics.median(times)
    return {
        "value": round(n_seq * T / med, 1),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"first {n_seq} of {inp['B']} sequences ({n_seq * T} token rows, same "
                   f"tensors), oracle hidden@W.T->log_softmax->gather->clip->autograd through "
                   f"the LM head in float32, median of {runs} runs after 1 warm-up, torch "
                   f"threads={threads}, os.cpu_count()={os.cpu_count()}"),
    }


def traffic_from_profiles(kernel_key, workload_key):
    """HBM bytes per launch from the committed rocprofv3 counter summary, if
    one exists for this kernel and workload (else None)."""

    f = ROOT / "profiles" / "hbm_traffic.json"
    if not f.exists():
        return None
    try:
        entry = json.loads(f.read_text())[kernel_key][workload_key]
        return entry["bytes_per_launch"]
    except (KeyError, ValueError, TypeError):
        return None


def timed_steps(step, steps, kernels):
    """Time `steps` calls of `step` by the wall clock, bracketed by device
    synchronisations, then run as many again with HIP events recorded around
    every launch of `kernels` (on the stream each is launched on).  Returns
    (seconds of the first loop, its last output, {kernel: [(start, end)]}):
    the events never sit inside the wall-clock loop."""

    import torch

    from rosellm_amd import _native as nat

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    timed = nat.time_calls(*kernels, capacity=steps * 32)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    nat.time_calls()
    return elapsed, out, timed


SAMPLE_ROWS = 256
SAMPLE_VARIANTS = {"default": dict(temperature=1.0, top_k=0, top_p=1.0, do_sample=True),
                   "topk50_topp0.9_T0.7": dict(temperature=0.7, top_k=50, top_p=0.9,
                                               do_sample=True),
                   "greedy": dict(temperature=1.0, top_k=0, top_p=1.0, do_sample=False)}


def bench_sample(args):
    """Rollout sampling: tokens/s of sample_next_token_batch over 256 rows of
    151936 bf16 logits (config 2's distribution), one call per step."""

    import numpy as np
    import torch

    from oracle import sampler_oracle as so
    from rosellm_amd import _native as nat
    from rosellm_amd.roseinfer import sample_next_token_batch

    device = torch.device("cuda", 0)
    B, V = SAMPLE_ROWS, 151936
    g = torch.Generator(device=device).manual_seed(args.seed)
    x = torch.randn(B, V, dtype=torch.bfloat16, device=device, generator=g).mul_(3.0)
    hot = torch.randint(0, V, (B,), device=device, generator=g)
    rows = torch.arange(0, B, 20, device=device)
    x[rows, hot[rows]] = (x[rows, hot[rows]].float() + 15.0).to(torch.bfloat16)
    results = {}
    for name, kw in SAMPLE_VARIANTS.items():
        for i in range(args.warmup):
            sample_next_token_batch(x, seed=args.seed, offset=i, **kw)
        offs = iter(range(100, 100 + 2 * args.steps))
        el, out, timed = timed_steps(
            lambda: sample_next_token_batch(x, seed=args.seed, offset=next(offs), **kw),
            args.steps, ["rrl_sample_logprobs"])
        kms = [s.elapsed_time(e) for s, e in timed["rrl_sample_logprobs"]]
        results[name] = dict(ms=el * 1e3 / args.steps, kernel_ms=sum(kms) / len(kms),
                             tokens=out.token_ids)
        log(f"[bench] sample {name}: {el * 1e3 / args.steps:.4f} ms/step, kernel "
            f"{results[name]['kernel_ms']:.4f} ms")
    head = results["default"]
    alg = B * (V * 2 + 8 + 4 + 4)  # one read of the logits; token + two log-probs out
    achieved = alg / (head["kernel_ms"] * 1e-3) / 1e9
    cpu = None
    if not args.skip_cpu:
        n = 16
        xc = x[:n].float().cpu().numpy()
        times = []
        for i in range(args.cpu_runs + 1):
            t0 = time.perf_counter()
            so.sample_rows(xc, temperature=1.0, top_k=0, top_p=1.0, do_sample=True,
                           seed=args.seed, offset=0)
            if i:
                times.append(time.perf_counter() - t0)
        med = statistics.median(times)
        cpu = {"value": round(n / med, 1), "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": f"first {n} of {B} rows, oracle inverse-CDF sampler in float64 NumPy "
                         f"(one thread), median of {args.cpu_runs} runs after 1 warm-up"}
    result = {
        "metric": "tokens/sec sampled with behaviour log-probs @151936 vocab (rollout side)",
        "value": round(B / (head["ms"] * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (config 2's logits distribution, generated on the GPU)",
        "config": {"workload": "Rollout sampling: 256 rows x V=151936 bf16 -> token + behaviour "
                               "log-probs (roseinfer/engine.py:1103-1171 defaults)",
                   "rows": B, "vocab": V, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "kernel": "rrl_sample_logprobs",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profiles("rrl_sample_logprobs", "sample-default"),
                     "kernel_ms": round(head["kernel_ms"], 4), "alg_bytes_per_launch": alg},
        "cpu_baseline": cpu,
        "variants": {k: {"ms_per_step": round(v["ms"], 4), "kernel_ms": round(v["kernel_ms"], 4),
                         "value": round(B / (v["ms"] * 1e-3), 1)}
                     for k, v in results.items() if k != "default"},
    }
    print(json.dumps(result), flush=True)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the path "
              "shards by whole GRPO groups with one scalar all-reduce per step, which "
              "is not run here.", file=sys.stderr)
        sys.exit(2)
    if args.steps is None:
        args.steps = 200 if args.config in ("c1", "sample") else 10
    if args.warmup is None:
        args.warmup = 20 if args.config in ("c1", "sample") else 2
    if args.config == "sample":
        bench_sample(args)
        return

    import torch

    from rosellm_amd import _native as nat

    device = torch.device("cuda", 0)
    cfg = CONFIGS[args.config]
    log(f"[bench] config {args.config} path {args.path}: generating inputs")
    t0 = time.perf_counter()
    with torch.no_grad():
        inp = make_inputs(cfg, device, args.seed)
    torch.cuda.synchronize()
    log(f"[bench] inputs ready in {time.perf_counter() - t0:.1f} s")
    N, V = inp["B"] * inp["T"], inp["V"]
    objective = cfg["objective"]
    if args.objective:
        if args.config != "c3":
            raise SystemExit("--objective applies to config c3")
        objective = args.objective
    cfg = dict(cfg, objective=objective)
    # GSPO needs every token's log-prob before any gradient: its fused entry is
    # the two-kernel composition (forward sweep, backward sweep).
    path = args.path if objective in ("clipped", "sapo") else "composed"
    if cfg.get("sft"):
        path = "fused"
    step = make_step(inp, cfg, path, objective)

    for i in range(args.warmup):
        step()
        torch.cuda.synchronize()
        log(f"[bench] warmup {i} done")

    kernels = (["rrl_fused_logprob_policy"] if path == "fused"
               else ["rrl_logprob_fwd", "rrl_logprob_bwd"])
    elapsed, out, timed = timed_steps(step, args.steps, kernels)
    ms_step = elapsed * 1e3 / args.steps
    tok_s = N / (elapsed / args.steps)
    in_b = (inp["hidden"] if cfg.get("lm_head") else inp["logits"]).element_size()
    # Rows one launch of the single-pass kernel processes, and their side data
    # (the SFT loss scores the B*(T-1) positions that have a next token).
    k_rows, side = (inp["B"] * (inp["T"] - 1), SFT_SIDE_BYTES) if cfg.get("sft") else (N, SIDE_BYTES)
    # Algorithmic bytes per launch of each timed entry point.
    alg = {
        # read logits + write dlogits, 8 target + 4 old + 4 advantage + 1 mask + 4 logp
        "rrl_fused_logprob_policy": k_rows * (V * (in_b + in_b) + side),
        # read logits, 8 target, write 4 logp + 4 lse
        "rrl_logprob_fwd": N * (V * in_b + 8 + 4 + 4),
        # read logits + write dlogits, 8 target + 4 lse + 4 logp + 4 g (the
        # logits read is narrowed to the rows with a non-zero g below)
        "rrl_logprob_bwd": N * (V * (in_b + in_b) + 8 + 4 + 4 + 4),
    }
    if path == "composed":
        # Rows whose d loss / d logp is exactly zero (masked, clipped or
        # zero-advantage tokens) are written as zeros without reading their
        # logits: count them on one extra, untimed step.
        probe = {}
        make_step(inp, cfg, path, objective, probe=probe)()
        torch.cuda.synchronize()
        active = probe["active"]
        alg["rrl_logprob_bwd"] = N * V * in_b + active * V * in_b + N * (8 + 4 + 4 + 4)
        log(f"[bench] backward reads the logits of {active} of {N} rows")
    kstats = {}
    for k in kernels:
        kms = [s.elapsed_time(e) for s, e in timed[k]]
        kstats[k] = sum(kms) / len(kms)
    kernel = max(kernels, key=lambda k: kstats[k])  # the dominant kernel
    k_avg = kstats[kernel]
    log(f"[bench] {args.steps} steps: {ms_step:.3f} ms/step, {tok_s / 1e6:.3f} M tok/s; "
        + ", ".join(f"{k} avg {v:.3f} ms" for k, v in kstats.items())
        + f"; loss {out.loss.item():.6g}")
    achieved = alg[kernel] / (k_avg * 1e-3) / 1e9
    workload_key = f"{args.config}-{path}" + (f"-{objective}" if args.config == "c3" else "")
    if cfg.get("lm_head"):
        # Config 5 is bound by the three GEMMs (hidden x W^T, dlogits x W,
        # dlogits^T x hidden): 3 x 2*N*H*V flops per step against the dense
        # bf16 MFMA peak; the row kernel's share is reported beside it.
        H = inp["hidden"].shape[-1]
        flops = 3 * 2 * N * H * V
        tflops = flops / (ms_step * 1e-3) / 1e12
        per_step = len(timed[kernel]) / args.steps  # row-kernel launches per step
        rows_launch = N / per_step
        alg_launch = (rows_launch * (V * (in_b + in_b) + SIDE_BYTES) if kernel != "rrl_logprob_fwd"
                      else rows_launch * (V * in_b + 16))
        k_gbs = alg_launch / (k_avg * 1e-3) / 1e9
        roofline = {
            "bound": "mfma",
            "kernel": "whole step (hipBLASLt GEMMs + " + kernel + ")",
            "achieved": round(tflops, 1),
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "traffic": None,
            "alg_flops_per_step": flops,
            "row_kernel": {"name": kernel, "launches_per_step": per_step,
                           "kernel_ms": round(k_avg, 4),
                           "ms_per_step": round(k_avg * per_step, 4),
                           "alg_bytes_per_launch": alg_launch,
                           "achieved_GBs": round(k_gbs, 1),
                           "frac_hbm": round(k_gbs / HBM_PEAK_GBS, 4)},
            "kernels_ms": {k: round(v, 4) for k, v in kstats.items()},
            "blas": str(torch.backends.cuda.preferred_blas_library()),
        }
    else:
        roofline = {
            "bound": "hbm",
            "kernel": kernel,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profiles(kernel, workload_key),
            "kernel_ms": round(k_avg, 4),
            "alg_bytes_per_launch": alg[kernel],
            "kernels_ms": {k: round(v, 4) for k, v in kstats.items()},
            # whole step against the algorithmic minimum of one logits read and
            # one dlogits write
            "step_frac": round(N * (V * 2 * in_b + side) / (ms_step * 1e-3) / 1e9
                               / HBM_PEAK_GBS, 4),
        }

    # The same step with skip_masked_rows=True (zero-weight rows are never
    # read); reported beside the exact-semantics headline, not as `value`.
    variants = {}

    def time_variant(vstep):
        """Warm-up, then the timed steps of a variant: (seconds, average
        duration of the dominant entry point in ms, last output)."""

        for _ in range(args.warmup):
            vstep()
        v_el, vout, vt = timed_steps(vstep, args.steps, kernels[:1])
        v_ms = [s.elapsed_time(e) for s, e in vt[kernels[0]]]
        return v_el, sum(v_ms) / len(v_ms), vout

    if (path == "fused" and objective == "clipped" and not args.no_variants
            and not cfg.get("lm_head")):
        v_el, v_k, vout = time_variant(make_step(inp, cfg, path, objective, skip_masked=True))
        assert vout.loss.item() == out.loss.item(), "skip_masked_rows changed the loss"
        n_active = int(inp["mask"].sum().item())
        v_alg = n_active * V * in_b + N * V * in_b + N * SIDE_BYTES
        variants["skip_masked_rows"] = {
            "value": round(N / (v_el / args.steps), 1),
            "ms_per_step": round(v_el * 1e3 / args.steps, 4),
            "kernel_ms": round(v_k, 4),
            "active_rows": n_active,
            "alg_bytes_per_launch": v_alg,
            "achieved": round(v_alg / (v_k * 1e-3) / 1e9, 1),
            "frac": round(v_alg / (v_k * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        }
        log(f"[bench] skip_masked_rows: {v_el * 1e3 / args.steps:.3f} ms/step, "
            f"{N / (v_el / args.steps) / 1e6:.3f} M tok/s, kernel {v_k:.3f} ms")

    if objective == "sapo" and not args.no_variants:
        # Config 4 is specified with tau_negative = 1.0; the reference's
        # default (tau_positive 1.0, tau_negative 1.05) is reported beside it.
        # Same bytes per step: the taus change only the per-token arithmetic.
        ref_kw = dict(tau_positive=1.0, tau_negative=1.05)
        v_el, v_k, _ = time_variant(make_step(inp, dict(cfg, kw=ref_kw), path, objective))
        v_alg = alg[kernels[0]]
        variants["reference_default_taus"] = {
            "kw": ref_kw,
            "value": round(N / (v_el / args.steps), 1),
            "ms_per_step": round(v_el * 1e3 / args.steps, 4),
            "kernel_ms": round(v_k, 4),
            "achieved": round(v_alg / (v_k * 1e-3) / 1e9, 1),
            "frac": round(v_alg / (v_k * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        }
        log(f"[bench] SAPO with the reference's default taus: {v_el * 1e3 / args.steps:.3f} "
            f"ms/step, {N / (v_el / args.steps) / 1e6:.3f} M tok/s, kernel {v_k:.3f} ms")

    if args.calibrate_copy:
        # Calibration kernel of known traffic for the HBM counters: a bf16 ->
        # float32 conversion of 2^30 random elements reads 2 GiB and writes
        # 4 GiB (a same-dtype copy would run as a DMA blit, invisible to the
        # counters; constant data can compress in the memory fabric).
        src = torch.randn(1 << 30, dtype=torch.bfloat16, device=device)
        dst = torch.empty(1 << 30, dtype=torch.float32, device=device)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] calibration conversion: {src.numel() * 2} B read, {dst.numel() * 4} B written")
        del src, dst

    cpu = None
    if not args.skip_cpu:
        n_seq = min(args.cpu_sample_seqs, inp["B"])
        cpu = cpu_baseline(inp, cfg, n_seq, args.cpu_runs)

    result = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"].replace("bfloat16", "bf16").replace("float32", "fp32"),
        "data": "synthetic (config distributions, generated on the GPU, seed 1234+i)",
        "config": {
            "workload": cfg["workload"],
            "objective": objective,
            "path": path,
            "sequences": inp["B"],
            "seq_len": inp["T"],
            "vocab": V,
            **({"hidden": inp["hidden"].shape[-1], "row_block": LM_HEAD_ROW_BLOCK}
               if cfg.get("lm_head") else {}),
            "tokens_per_step": N,
            "parallelism": "none (1 GPU)",
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    if variants:
        result["variants"] = variants
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
