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

After the headline the same run times every other configuration and reports
it under ``variants`` (each in its own try/except; an error string replaces a
failed one): C1, C3 with GSPO and with GSPO-token, C4 (GAE + whitening + SAPO,
dlogits in place: its logits are regenerated from their seed before every
step, outside the step's events, so every step runs on the config's data),
SFT, the rollout sampler and C5.

``--config c5`` is the fused LM-head step: hidden [256x1024, 1024] bf16 and
an LM-head weight [151936, 1024] bf16 -> log-probs -> clipped objective ->
d hidden and d weight, through ``fused_linear_policy_loss`` on the
hand-written MFMA kernels (``--path composed``: F.linear,
gather_token_logprobs, clipped_policy_loss, autograd).  Its roofline is
MFMA-bound: the reference's three products, 3 x 2*N*H*V = 244.7 TFLOP per
step, against the dense bf16 peak.

``--config sample`` is the rollout side: one decode step of 256 rows x
151936 bf16 logits -> next token + behaviour log-probs
(``rosellm_amd.roseinfer.sample_next_token_batch``, roseinfer/engine.py:
1103-1171 defaults T = 1, top_k = 0, top_p = 1; a top-k/top-p variant beside it).

``--config sft`` is the supervised next-token cross-entropy of the model
forwards (rosetrainer/model.py:643-649) on config 2's logits, labels = the
sampled tokens: ``rosellm_amd.rosetrainer.causal_lm_loss`` (the same
single-pass row kernel, objective NLL) -> backward to bf16 dlogits.

Prints one JSON line (rank 0): value = tokens/s over all B*T positions (the
wall clock over the timed steps; the median of the per-step event times is
beside it), ``roofline`` for the dominant kernel (HIP events around its
entry point over a second pass of the timed steps; algorithmic bytes
N*(V*(2+2) + 21) for the row kernels) and ``cpu_baseline``: the oracle's
PyTorch-CPU composition timed on a self-contained sub-batch (C1 whole,
C2/C3/SFT 16 sequences = 2 groups of 8, C4 2 x 8192, C5 16 sequences), with
the same sub-batch run through the HIP path in the same run as its parity
batch.
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
# Config 5's default (chunked) LM head: the library GEMMs, timed by HIP events
# around each call, and the row kernels between them.
LM_CHUNKED_KERNELS = ["lm_logits_gemm", "lm_dhidden_gemm", "lm_dweight_gemm",
                      "rrl_fused_logprob_policy", "rrl_logprob_fwd"]
LM_GEMMS = LM_CHUNKED_KERNELS[:3]
# impl="tiles": the hand-written MFMA kernels
LM_TILE_KERNELS = ["rrl_lm_head_fwd", "rrl_lm_head_dweight", "rrl_lm_head_dhidden"]
MFMA_BF16_PEAK_TFLOPS = 2500.0
# Sequences of the CPU plan's sub-batch per config (C1 whole; C4's are 8192 long).
CPU_SEQS = {"c1": 32, "c2": 16, "c3": 16, "sft": 16, "c4": 2, "c5": 16}
# Configurations timed after the headline, reported under "variants".
VARIANTS = ["c1", "c3", "c3_gspo_token", "c4", "c4_tau_default", "sft", "sample", "c5"]


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
    p.add_argument("--cpu-sample-seqs", type=int, default=None,
                   help="sequences of the batch timed on the CPU oracle (default: the CPU "
                        "plan's sub-batch of the config)")
    p.add_argument("--cpu-runs", type=int, default=3)
    p.add_argument("--skip-cpu", action="store_true")
    p.add_argument("--no-variants", action="store_true",
                   help="time the headline configuration only, without its skip_masked_rows "
                        "variant")
    p.add_argument("--headline-only", action="store_true",
                   help="time the headline configuration and its own variants, not the other "
                        "configurations")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="after the headline, launch two conversions of known traffic (HBM counter "
                        "calibration)")
    p.add_argument("--seed", type=int, default=1234)
    return p.parse_args()


def fill_logits(logits, cfg, device, seed):
    """The config's logits, written into ``logits`` [B, T, V] from generators
    seeded seed + 0, 1, 2 (the same values on every call)."""

    import torch

    V = logits.shape[-1]
    gens = [torch.Generator(device=device).manual_seed(seed + i) for i in range(3)]
    torch.randn(logits.shape, dtype=logits.dtype, device=device, generator=gens[0], out=logits)
    logits.mul_(cfg["sigma"])
    if cfg["hot"] > 0:
        flat = logits.view(-1, V)
        hot_rows = torch.nonzero(torch.rand(flat.shape[0], device=device, generator=gens[1])
                                 < cfg["hot"]).reshape(-1)
        hot_cols = torch.randint(0, V, (hot_rows.numel(),), device=device, generator=gens[2])
        flat[hot_rows, hot_cols] = (flat[hot_rows, hot_cols].float() + 15.0).to(logits.dtype)


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
        logits = torch.empty(B, T, V, dtype=dtype, device=device)
        fill_logits(logits, cfg, device, seed)
        flat = logits.view(-1, V)
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


def make_step(inp, cfg, path, objective, skip_masked=False, probe=None, impl="auto"):
    """One timed step of the config's training-step hot path.  With ``probe``
    (a dict; composed path only, never in a timed step) the step also records
    how many token rows receive a non-zero d loss / d logp: the backward
    kernel reads the logits of those rows only.  ``impl`` picks config 5's
    LM-head implementation ("auto" = chunked, or "tiles")."""

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
                                                 skip_masked_rows=skip_masked, impl=impl,
                                                 **kw)
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
        # overwrite the logits (logits + dlogits would need 318.6 GB); the
        # timing loops regenerate the logits from their seed before every
        # step (prepare_step), outside the step's events.
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


def cpu_info():
    """Host facts recorded beside every CPU figure."""

    import torch

    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(),
            "cpu_model": model}


def _median_runs(fn, runs, what):
    """Run fn() 1 + runs times (the first a warm-up): (median seconds, last output)."""

    times, out = [], None
    for i in range(runs + 1):
        t0 = time.perf_counter()
        out = fn()
        dt = time.perf_counter() - t0
        if i > 0:
            times.append(dt)
        log(f"[bench] cpu oracle {what} run {i}: {dt:.2f} s")
    return statistics.median(times), out


def _err(got, want, chunk=1024):
    """Largest absolute difference, largest |want|, and the relative L2 norm of
    the difference, accumulated in float64 over row chunks (host memory stays
    a few chunks)."""

    g2 = got.detach().reshape(-1, got.shape[-1])
    w2 = want.detach().reshape(-1, want.shape[-1])
    mx = mw = ss_d = ss_w = 0.0
    for r0 in range(0, g2.shape[0], chunk):
        g = g2[r0:r0 + chunk].cpu().double()
        w = w2[r0:r0 + chunk].cpu().double()
        d = g - w
        mx = max(mx, float(d.abs().max()))
        mw = max(mw, float(w.abs().max()))
        ss_d += float((d * d).sum())
        ss_w += float((w * w).sum())
    return {"max_abs_err": mx, "max_abs": mw,
            "rel_l2": math.sqrt(ss_d / ss_w) if ss_w > 0 else math.sqrt(ss_d)}


def cpu_baseline(inp, cfg, name, objective, path, n_seq, runs):
    """The oracle's PyTorch-CPU composition (log_softmax -> gather -> objective
    -> autograd), op for op the reference's, timed on the first n_seq
    sequences (for C2/C3/SFT: 2 whole groups of 8, self-contained), and the
    same sub-batch through the HIP path as its parity batch."""

    import torch

    from oracle import roserlhf_oracle as o
    from rosellm_amd import roserlhf as R

    T = inp["T"]
    if cfg.get("lm_head"):
        return cpu_baseline_lm_head(inp, cfg, n_seq, runs)
    if cfg.get("sft"):
        return cpu_baseline_sft(inp, n_seq, runs)
    x = inp["logits"].detach()[:n_seq].cpu()
    t = inp["actions"][:n_seq].cpu()
    old = inp["old"][:n_seq].cpu()
    mask = inp["mask"][:n_seq].cpu()
    if objective == "sapo":
        adv, _ = o.gae(inp["rewards"][:n_seq].cpu(), inp["values"][:n_seq].cpu(), gamma=1.0,
                       gae_lambda=0.95, valid_mask=mask)
        adv = o.masked_whiten(adv, mask)
    else:
        seq_adv = o.group_standardize(inp["rewards"].cpu()).reshape(-1)[:n_seq]
        adv = seq_adv if objective == "gspo" else seq_adv[:, None].expand(n_seq, T)
    kind = {"clipped": "ppo"}.get(objective, objective)
    med, (out_c, _lp, dl_c) = _median_runs(
        lambda: o.policy_step(kind, x, t, old, adv, mask, **cfg["kw"]), runs, name)
    # the same sub-batch on the GPU (a copy of its logits: C4 works in place)
    dev = inp["logits"].device
    xg = inp["logits"].detach()[:n_seq].clone().requires_grad_()
    d = lambda z: z.to(dev)  # noqa: E731
    if path == "fused":
        out_g = R.fused_policy_loss(xg, d(t), d(old), d(adv), d(mask), objective=objective,
                                    **cfg["kw"])
    else:
        fn = {"clipped": R.clipped_policy_loss, "gspo": R.gspo_policy_loss,
              "gspo_token": R.gspo_token_policy_loss, "sapo": R.sapo_policy_loss}[objective]
        out_g = fn(R.gather_token_logprobs(xg, d(t)), d(old), d(adv), d(mask), **cfg["kw"])
    out_g.loss.backward()
    torch.cuda.synchronize()
    lc, lg = float(out_c["loss"]), float(out_g.loss)
    parity = {"loss_cpu": lc, "loss_gpu": lg,
              "loss_rel_err": abs(lg - lc) / max(abs(lc), 1e-30),
              "dlogits": _err(xg.grad, dl_c)}
    del xg, dl_c
    rows = n_seq * T
    return {
        "value": round(rows / med, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
        "kind": "port", "median_s": round(med, 4),
        "sample": (f"first {n_seq} of {inp['B']} sequences ({rows} token rows, the same "
                   f"tensors copied from the GPU), oracle log_softmax->gather->{objective}->"
                   f"autograd on the fp32 upcast, median of {runs} runs after 1 warm-up"),
        **cpu_info(), "gpu_parity": parity,
    }


def cpu_baseline_sft(inp, n_seq, runs):
    """SFT loss on the CPU: the oracle's shift -> log_softmax -> gather ->
    mean -> autograd on the float32 upcast of the first n_seq sequences; the
    same sub-batch through the HIP path as its parity batch."""

    import torch

    from oracle import roserlhf_oracle as o
    from rosellm_amd import rosetrainer as RT

    T = inp["T"]
    x = inp["logits"].detach()[:n_seq].cpu()
    t = inp["actions"][:n_seq].cpu()
    med, (loss_c, dl_c) = _median_runs(lambda: o.sft_step(x, t, causal=True), runs, "sft")
    xg = inp["logits"].detach()[:n_seq].clone().requires_grad_()
    loss_g = RT.causal_lm_loss(xg, t.to(xg.device))
    loss_g.backward()
    torch.cuda.synchronize()
    lc, lg = float(loss_c), float(loss_g)
    parity = {"loss_cpu": lc, "loss_gpu": lg,
              "loss_rel_err": abs(lg - lc) / max(abs(lc), 1e-30),
              "dlogits": _err(xg.grad, dl_c)}
    del xg, dl_c
    rows = n_seq * T
    return {
        "value": round(rows / med, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
        "kind": "port", "median_s": round(med, 4),
        "sample": (f"first {n_seq} of {inp['B']} sequences ({rows} token rows, the same "
                   f"tensors), oracle shift->log_softmax->gather->mean->autograd on the fp32 "
                   f"upcast, median of {runs} runs after 1 warm-up"),
        **cpu_info(), "gpu_parity": parity,
    }


def cpu_baseline_lm_head(inp, cfg, n_seq, runs):
    """Config 5 on the CPU: the reference chain (hidden @ W.T, log_softmax,
    gather, clipped objective, autograd back through the linear map) in
    float32 on the first n_seq sequences; the same sub-batch through the HIP
    path as its parity batch."""

    import torch

    from oracle import roserlhf_oracle as o
    from rosellm_amd import roserlhf as R

    T = inp["T"]
    h = inp["hidden"].detach()[:n_seq].cpu().float()
    w = inp["weight"].detach().cpu().float()
    t = inp["actions"][:n_seq].cpu()
    old = inp["old"][:n_seq].cpu()
    mask = inp["mask"][:n_seq].cpu()
    seq_adv = o.group_standardize(inp["rewards"].cpu()).reshape(-1)[:n_seq]
    adv = seq_adv[:, None].expand(n_seq, T)

    def run():
        x = h @ w.t()
        return o.lm_head_step("ppo", h, w, x, t, old, adv, mask, **cfg["kw"])

    med, (out_c, _lp, dh_c, dw_c) = _median_runs(run, runs, "c5")
    dev = inp["hidden"].device
    hg = inp["hidden"].detach()[:n_seq].clone().requires_grad_()
    wg = inp["weight"].detach().clone().requires_grad_()
    d = lambda z: z.to(dev)  # noqa: E731
    out_g = R.fused_linear_policy_loss(hg, wg, d(t), d(old), d(adv), d(mask), **cfg["kw"])
    out_g.loss.backward()
    torch.cuda.synchronize()
    lc, lg = float(out_c["loss"]), float(out_g.loss)
    parity = {"loss_cpu": lc, "loss_gpu": lg,
              "loss_rel_err": abs(lg - lc) / max(abs(lc), 1e-30),
              "dhidden": _err(hg.grad, dh_c), "dweight": _err(wg.grad, dw_c)}
    del hg, wg
    # The reference's own chain on the GPU in bf16 (F.linear, log_softmax of
    # the float32 upcast, gather, clipped objective, autograd: bf16 dlogits,
    # bf16 products), against the same float32 CPU chain.
    import torch.nn.functional as F

    hr = inp["hidden"].detach()[:n_seq].clone().requires_grad_()
    wr = inp["weight"].detach().clone().requires_grad_()
    x = F.linear(hr, wr)
    lp = F.log_softmax(x.float(), dim=-1).gather(-1, d(t).unsqueeze(-1)).squeeze(-1)
    del x
    out_r = o.ppo_clip(lp, d(old).float(), d(adv).float(), d(mask), **cfg["kw"])
    out_r["loss"].backward()
    torch.cuda.synchronize()
    parity["torch_bf16_chain"] = {
        "loss_rel_err": abs(float(out_r["loss"]) - lc) / max(abs(lc), 1e-30),
        "dhidden": _err(hr.grad, dh_c), "dweight": _err(wr.grad, dw_c),
        "note": "F.linear -> log_softmax(float32) -> gather -> clip -> autograd on the GPU "
                "in bf16, against the float32 CPU chain"}
    del hr, wr, lp, out_r
    torch.cuda.empty_cache()
    rows = n_seq * T
    return {
        "value": round(rows / med, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
        "kind": "port", "median_s": round(med, 4),
        "sample": (f"first {n_seq} of {inp['B']} sequences ({rows} token rows, same "
                   f"tensors), oracle hidden@W.T->log_softmax->gather->clip->autograd through "
                   f"the LM head in float32, median of {runs} runs after 1 warm-up"),
        **cpu_info(), "gpu_parity": parity,
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


def timed_steps(step, steps, kernels, prepare=None):
    """Time `steps` calls of `step`: a wall-clock loop bracketed by device
    synchronisations, with one event recorded between consecutive steps (the
    per-step times), then as many steps again with HIP events recorded around
    every launch of `kernels` (on the stream each is launched on).  With
    `prepare` (run before each step, outside its events) the wall clock would
    include it: only the per-step events time the steps.  Returns a dict:
    wall_s (None with prepare), step_ms (list), out (the last output), launches
    ({kernel: [(start, end)]})."""

    import torch

    from rosellm_amd import _native as nat

    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * steps)]
    host = [0.0] * (steps + 1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    host[0] = t0
    out = None
    for i in range(steps):
        if prepare is not None:
            prepare()
        ev[2 * i].record()
        out = step()
        ev[2 * i + 1].record()
        host[i + 1] = time.perf_counter()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    wall = None if prepare is not None else t1 - t0
    # host time from one step() call's return to the next one's (the last one
    # up to the closing synchronisation)
    host_ms = [(host[i + 1] - host[i]) * 1e3 for i in range(steps)]
    host_ms[-1] += (t1 - host[steps]) * 1e3
    if prepare is None:
        # consecutive steps: the time from one step's start to the next one's
        step_ms = [ev[2 * i].elapsed_time(ev[2 * i + 2]) for i in range(steps - 1)]
        step_ms.append(ev[2 * steps - 2].elapsed_time(ev[2 * steps - 1]))
    else:
        step_ms = [ev[2 * i].elapsed_time(ev[2 * i + 1]) for i in range(steps)]
    timed = nat.time_calls(*kernels, capacity=steps * 64)
    for _ in range(steps):
        if prepare is not None:
            prepare()
        step()
    torch.cuda.synchronize()
    nat.time_calls()
    return {"wall_s": wall, "step_ms": step_ms, "host_ms": host_ms, "out": out,
            "launches": timed}


def kernel_stats(launches, kernels, steps):
    """{kernel: (average ms per launch, launches per step)} of the recorded
    launches (kernels never launched are left out)."""

    stats = {}
    for k in kernels:
        kms = [s.elapsed_time(e) for s, e in launches.get(k, [])]
        if kms:
            stats[k] = (sum(kms) / len(kms), len(kms) / steps)
    return stats


def measure_config(name, args, device, steps, warmup, with_cpu, cpu_seqs=None,
                   skip_masked_variant=False):
    """One configuration (a key of CONFIGS, or "c3_gspo_token"): inputs,
    warm-up, timed steps, the roofline of its dominant kernel and, with
    with_cpu, the CPU baseline with its GPU parity batch.  Returns the
    headline-format result dict."""

    import torch

    objective_override = None
    kw_override = None
    if name == "c3_gspo_token":
        name, objective_override = "c3", "gspo_token"
    elif name == "c4_tau_default":
        # SAPO at the reference's default temperatures (losses.py:361-362)
        name, kw_override = "c4", dict(tau_positive=1.0, tau_negative=1.05)
    cfg = CONFIGS[name]
    log(f"[bench] config {name}{'/' + objective_override if objective_override else ''}: "
        f"generating inputs")
    t0 = time.perf_counter()
    with torch.no_grad():
        inp = make_inputs(cfg, device, args.seed)
    torch.cuda.synchronize()
    log(f"[bench] inputs ready in {time.perf_counter() - t0:.1f} s")
    N, V = inp["B"] * inp["T"], inp["V"]
    objective = objective_override or cfg["objective"]
    cfg = dict(cfg, objective=objective)
    if objective_override == "gspo_token":
        cfg["workload"] = ("C3: GSPO-token objective fwd+bwd (losses.py:276-352), 256x1024 "
                           "tokens, V=151936 bf16")
    if kw_override is not None:
        cfg["kw"] = dict(cfg["kw"], **kw_override)
        cfg["workload"] = cfg["workload"] + ", SAPO tau (1.0, 1.05) (reference defaults)"
    # GSPO needs every token's log-prob before any gradient: its fused entry is
    # a forward sweep and a backward sweep (rrl_logprob_fwd, rrl_logprob_bwd).
    gspo_like = objective in ("gspo", "gspo_token")
    path = args.path
    if cfg.get("sft"):
        path = "fused"
    step = make_step(inp, cfg, path, objective)
    prepare = None
    if objective == "sapo":
        # C4 works in place: the logits are regenerated before each step.
        prepare = lambda: fill_logits(inp["logits"].data, cfg, device, args.seed)  # noqa: E731

    for i in range(warmup):
        if prepare is not None:
            prepare()
        step()
        torch.cuda.synchronize()
    log(f"[bench] {warmup} warm-up steps done")

    if cfg.get("lm_head"):
        kernels = list(LM_CHUNKED_KERNELS)
    elif path == "fused" and not gspo_like:
        kernels = ["rrl_fused_logprob_policy"]
    else:
        kernels = ["rrl_logprob_fwd", "rrl_logprob_bwd"]
    res = timed_steps(step, steps, kernels, prepare)
    step_ms = res["step_ms"]
    ms_step = (res["wall_s"] * 1e3 / steps if res["wall_s"] is not None
               else sum(step_ms) / len(step_ms))
    ms_median = statistics.median(step_ms)
    out = res["out"]
    tok_s = N / (ms_step * 1e-3)
    in_b = (inp["hidden"] if cfg.get("lm_head") else inp["logits"]).element_size()
    k_rows, side = ((inp["B"] * (inp["T"] - 1), SFT_SIDE_BYTES) if cfg.get("sft")
                    else (N, SIDE_BYTES))
    alg = {
        # read logits + write dlogits, 8 target + 4 old + 4 advantage + 1 mask + 4 logp
        "rrl_fused_logprob_policy": k_rows * (V * (in_b + in_b) + side),
        # read logits, 8 target, write 4 logp + 4 lse
        "rrl_logprob_fwd": N * (V * in_b + 8 + 4 + 4),
        # read logits + write dlogits, 8 target + 4 lse + 4 logp + 4 g (the
        # logits read is narrowed to the rows with a non-zero g below)
        "rrl_logprob_bwd": N * (V * (in_b + in_b) + 8 + 4 + 4 + 4),
    }
    active = None
    if (path == "composed" or gspo_like) and not cfg.get("lm_head"):
        # Rows whose d loss / d logp is exactly zero (masked, clipped or
        # zero-advantage tokens) are written as zeros without reading their
        # logits: count them on one extra, untimed step of the composition.
        probe = {}
        make_step(inp, cfg, "composed", objective, probe=probe)()
        torch.cuda.synchronize()
        active = probe["active"]
        alg["rrl_logprob_bwd"] = N * V * in_b + active * V * in_b + N * (8 + 4 + 4 + 4)
        log(f"[bench] backward reads the logits of {active} of {N} rows")
    kstats = kernel_stats(res["launches"], kernels, steps)
    kernels = [k for k in kernels if k in kstats]
    kernel = max(kernels, key=lambda k: kstats[k][0] * kstats[k][1])  # the dominant kernel
    k_avg = kstats[kernel][0]
    log(f"[bench] {steps} steps: {ms_step:.3f} ms/step (median {ms_median:.3f}), "
        f"{tok_s / 1e6:.3f} M tok/s; "
        + ", ".join(f"{k} avg {v[0]:.3f} ms" for k, v in kstats.items())
        + f"; loss {out.loss.item():.6g}")
    workload_key = f"{name}-{path}" + (f"-{objective}" if name == "c3" else "")
    if cfg.get("lm_head"):
        roofline = lm_head_roofline(inp, kstats, ms_step)
    else:
        achieved = alg[kernel] / (k_avg * 1e-3) / 1e9
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
            "kernels_ms": {k: round(v[0], 4) for k, v in kstats.items()},
            # whole step against the algorithmic minimum of one logits read and
            # one dlogits write
            "step_frac": round(k_rows * (V * 2 * in_b + side) / (ms_step * 1e-3) / 1e9
                               / HBM_PEAK_GBS, 4),
        }

    variants = {}
    if skip_masked_variant and path == "fused" and gspo_like:
        # GSPO with skip_masked_rows=True: the forward sweep reads the masked-in
        # rows only; the backward reads the rows with a non-zero gradient and
        # writes every dlogits row.  Bytes it moves: those reads, one dlogits
        # write, and the side data of both sweeps.
        vstep = make_step(inp, cfg, path, objective, skip_masked=True)
        for _ in range(warmup):
            vstep()
        vk = ["rrl_logprob_fwd_masked", "rrl_logprob_bwd"]
        vres = timed_steps(vstep, steps, vk)
        v_el = vres["wall_s"]
        vms = {k: [s.elapsed_time(e) for s, e in vres["launches"][k]] for k in vk}
        vavg = {k: sum(v) / len(v) for k, v in vms.items()}
        assert torch.equal(vres["out"].loss, out.loss), "skip_masked_rows changed the loss"
        n_active = int((inp["mask"] != 0).sum().item())
        v_alg = {"rrl_logprob_fwd_masked": n_active * V * in_b + N * (8 + 1 + 4 + 4),
                 "rrl_logprob_bwd": active * V * in_b + N * V * in_b + N * (8 + 4 + 4 + 4)}
        k_sum = sum(vavg.values())
        step_alg = sum(v_alg.values())
        variants["skip_masked_rows"] = {
            "value": round(N / (v_el / steps), 1),
            "ms_per_step": round(v_el * 1e3 / steps, 4),
            "ms_per_step_median": round(statistics.median(vres["step_ms"]), 4),
            "kernels_ms": {k: round(v, 4) for k, v in vavg.items()},
            "mask_active_rows": n_active,
            "grad_active_rows": active,
            "alg_bytes_per_step": step_alg,
            "alg_bytes_per_launch": v_alg,
            "achieved": round(step_alg / (k_sum * 1e-3) / 1e9, 1),
            "frac": round(step_alg / (k_sum * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "note": "achieved = both sweeps' bytes over both kernels' time",
            # the single-sweep algorithmic bytes of a step that skips masked
            # rows (one read of the masked-in rows, one dlogits write, 21 B of
            # side data per token) over the step time; GSPO's sequence ratio
            # needs a second read of the rows with a gradient, which this
            # figure leaves out
            "baseline_skip_bytes": n_active * V * in_b + N * V * in_b + N * SIDE_BYTES,
            "baseline_skip_frac": round((n_active * V * in_b + N * V * in_b + N * SIDE_BYTES)
                                        / (v_el / steps) / 1e9 / HBM_PEAK_GBS, 4),
        }
        log(f"[bench] skip_masked_rows: {v_el * 1e3 / steps:.3f} ms/step, kernels "
            + ", ".join(f"{k} {v:.3f} ms" for k, v in vavg.items()))
    if skip_masked_variant and path == "fused" and cfg.get("lm_head"):
        # Config 5 with skip_masked_rows=True: the tokens of zero mask weight
        # are never formed (no logits, no log-sum-exp); loss and gradients are
        # those of the headline step.
        vstep = make_step(inp, cfg, path, objective, skip_masked=True)
        for _ in range(warmup):
            vstep()
        vres = timed_steps(vstep, steps, LM_CHUNKED_KERNELS)
        v_ms = vres["wall_s"] * 1e3 / steps
        assert vres["out"].loss.item() == out.loss.item(), "skip_masked_rows changed the loss"
        vroof = lm_head_roofline(inp, kernel_stats(vres["launches"], LM_CHUNKED_KERNELS, steps),
                                 v_ms, skip=True)
        variants["skip_masked_rows"] = {
            "value": round(N / (v_ms * 1e-3), 1),
            "ms_per_step": round(v_ms, 4),
            "ms_per_step_median": round(statistics.median(vres["step_ms"]), 4),
            "step": vroof["step"],
            "kernels": vroof["kernels"],
            "other_ms_per_step": vroof["other_ms_per_step"],
            "note": "tokens of zero mask weight never formed; step frac on the model's "
                    "3*2*N*H*V flops",
        }
        del vstep, vres
        log(f"[bench] skip_masked_rows: {v_ms:.3f} ms/step")
        # impl="tiles": the hand-written MFMA kernels, no logits beyond one tile
        tstep = make_step(inp, cfg, path, objective, impl="tiles")
        for _ in range(warmup):
            tstep()
        tres = timed_steps(tstep, steps, LM_TILE_KERNELS)
        t_ms = tres["wall_s"] * 1e3 / steps
        troof = lm_head_tiles_roofline(inp, kernel_stats(tres["launches"], LM_TILE_KERNELS,
                                                         steps), t_ms)
        variants["tiles"] = {
            "value": round(N / (t_ms * 1e-3), 1),
            "ms_per_step": round(t_ms, 4),
            "ms_per_step_median": round(statistics.median(tres["step_ms"]), 4),
            "loss": tres["out"].loss.item(),
            "roofline": troof,
            "note": "impl='tiles': the hand-written MFMA LM-head kernels",
        }
        del tstep, tres
        log(f"[bench] tiles: {t_ms:.3f} ms/step, "
            + ", ".join(f"{k} {v:.3f} ms" for k, v in troof["kernels_ms"].items()))
    if skip_masked_variant and path == "fused" and objective == "clipped" \
            and not cfg.get("lm_head"):
        # The same step with skip_masked_rows=True (zero-weight rows are never
        # read); reported beside the exact-semantics headline, not as `value`.
        vstep = make_step(inp, cfg, path, objective, skip_masked=True)
        for _ in range(warmup):
            vstep()
        vres = timed_steps(vstep, steps, kernels[:1])
        v_el = vres["wall_s"]
        v_ms = [s.elapsed_time(e) for s, e in vres["launches"][kernels[0]]]
        v_k = sum(v_ms) / len(v_ms)
        assert vres["out"].loss.item() == out.loss.item(), "skip_masked_rows changed the loss"
        n_active = int(inp["mask"].sum().item())
        v_alg = n_active * V * in_b + N * V * in_b + N * SIDE_BYTES
        variants["skip_masked_rows"] = {
            "value": round(N / (v_el / steps), 1),
            "ms_per_step": round(v_el * 1e3 / steps, 4),
            "ms_per_step_median": round(statistics.median(vres["step_ms"]), 4),
            "kernel_ms": round(v_k, 4),
            "active_rows": n_active,
            "alg_bytes_per_launch": v_alg,
            "achieved": round(v_alg / (v_k * 1e-3) / 1e9, 1),
            "frac": round(v_alg / (v_k * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        }
        log(f"[bench] skip_masked_rows: {v_el * 1e3 / steps:.3f} ms/step, "
            f"{N / (v_el / steps) / 1e6:.3f} M tok/s, kernel {v_k:.3f} ms")

    cpu = None
    if with_cpu:
        if prepare is not None:
            prepare()  # C4: the config's logits, not the last step's dlogits
        n_seq = min(cpu_seqs or CPU_SEQS.get(name, 16), inp["B"])
        cpu = cpu_baseline(inp, cfg, name, objective, path, n_seq, args.cpu_runs)

    result = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_step, 4),
        "ms_per_step_median": round(ms_median, 4),
        "step_time": ("wall clock over the timed steps" if res["wall_s"] is not None else
                      "mean of per-step events (the logits are regenerated between steps)"),
        # every timed step: device time from its start to the next step's
        # start (events), and the host's time between step() returns
        "per_step_ms": {"device": [round(v, 3) for v in step_ms],
                        "host": [round(v, 3) for v in res["host_ms"]]},
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
            **({"hidden": inp["hidden"].shape[-1]} if cfg.get("lm_head") else {}),
            "tokens_per_step": N,
            "parallelism": "none (1 GPU)",
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    if variants:
        result["variants"] = variants
    return result


def lm_head_roofline(inp, kstats, ms_step, skip=False):
    """Config 5 on the chunked LM head: the step against the dense bf16 MFMA
    peak on the reference's three products (3 x 2*N*H*V, the model's flops);
    each GEMM's flops (logits of every token, or of the masked-in tokens
    with ``skip``; d hidden and d weight of the masked-in tokens) over its
    launches' time; each row kernel's algorithmic bytes (the fused kernel
    reads a masked-in row's bf16 logits and writes its bf16 dlogits in place;
    the log-prob pass reads the other rows) over its launches' time.  The
    roofline is the GEMM with the most time per step."""

    N = inp["B"] * inp["T"]
    V, H = inp["V"], inp["hidden"].shape[-1]
    in_b = inp["hidden"].element_size()
    n_act = int((inp["mask"] != 0).sum().item())
    rows_fwd = n_act if skip else N
    flops = {"lm_logits_gemm": 2 * rows_fwd * H * V, "lm_dhidden_gemm": 2 * n_act * H * V,
             "lm_dweight_gemm": 2 * n_act * H * V}
    hbm = {"rrl_fused_logprob_policy": n_act * (V * (in_b + in_b) + SIDE_BYTES + 4),
           "rrl_logprob_fwd": (rows_fwd - n_act) * (V * in_b + 8 + 4 + 4)}
    per = {}
    timed_ms = 0.0
    for k, (avg, per_step) in kstats.items():
        ms = avg * per_step
        timed_ms += ms
        e = {"ms_per_launch": round(avg, 4), "launches_per_step": round(per_step, 3),
             "ms_per_step": round(ms, 3)}
        if k in flops:
            tf = flops[k] / (ms * 1e-3) / 1e12
            e.update(flops_per_step=flops[k], TFLOPs=round(tf, 1),
                     frac=round(tf / MFMA_BF16_PEAK_TFLOPS, 4))
        elif k in hbm:
            gbs = hbm[k] / (ms * 1e-3) / 1e9
            e.update(alg_bytes_per_step=hbm[k], GBs=round(gbs, 1),
                     frac=round(gbs / HBM_PEAK_GBS, 4))
        per[k] = e
    gemms = [k for k in LM_GEMMS if k in kstats]
    dom = max(gemms, key=lambda k: per[k]["ms_per_step"])
    avg, per_step = kstats[dom]
    model = 3 * 2 * N * H * V
    step_tf = model / (ms_step * 1e-3) / 1e12
    achieved = flops[dom] / (avg * per_step * 1e-3) / 1e12
    return {
        "bound": "mfma",
        "kernel": dom,
        "achieved": round(achieved, 1),
        "peak": MFMA_BF16_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
        "traffic": None,
        "kernel_ms": round(avg, 4),
        # launches differ in rows (row blocks of 16384 tokens and the last,
        # shorter one): the mean over the step's launches
        "alg_flops_per_launch": round(flops[dom] / per_step),
        "step": {"model_flops": model, "achieved_TFLOPs": round(step_tf, 1),
                 "frac": round(step_tf / MFMA_BF16_PEAK_TFLOPS, 4),
                 "note": "the reference's three products 3*2*N*H*V over the step time"},
        "kernels": per,
        "other_ms_per_step": round(ms_step - timed_ms, 3),
        "active_rows": n_act,
        "kernels_ms": {k: round(v[0], 4) for k, v in kstats.items()},
    }


def lm_head_tiles_roofline(inp, kstats, ms_step):
    """Config 5 on the hand-written tile kernels (impl="tiles"): the step
    against the dense bf16 MFMA peak on the reference's three products
    (3 x 2*N*H*V, the model's flops), and each kernel's executed flops (the
    work skipping is exact: blocks of 64 tokens none of which needs obar run
    the log-sum-exp pass only, and the dW pass visits the 32-token tiles
    holding a token with a non-zero gradient)."""

    N = inp["B"] * inp["T"]
    V, H = inp["V"], inp["hidden"].shape[-1]
    mask = inp["mask"].reshape(-1)
    need_blocks = int(mask[: (N // 64) * 64].reshape(-1, 64).any(dim=1).sum().item())
    flops_model = 3 * 2 * N * H * V
    fwd_exec = 2 * N * H * V + 2 * need_blocks * 64 * H * V
    # tiles with a non-zero gradient: at most the tiles holding a masked-in token
    act_tiles = int(mask[: (N // 32) * 32].reshape(-1, 32).any(dim=1).sum().item())
    dw_exec = 2 * 2 * act_tiles * 32 * H * V
    fwd_ms = kstats["rrl_lm_head_fwd"][0]
    dw_ms = kstats["rrl_lm_head_dweight"][0]
    step_tf = flops_model / (ms_step * 1e-3) / 1e12
    fwd_tf = fwd_exec / (fwd_ms * 1e-3) / 1e12
    return {
        "bound": "mfma",
        "kernel": "rrl_lm_head_fwd",
        "achieved": round(fwd_tf, 1),
        "peak": MFMA_BF16_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(fwd_tf / MFMA_BF16_PEAK_TFLOPS, 4),
        "traffic": None,
        "kernel_ms": round(fwd_ms, 4),
        "alg_flops_per_launch": fwd_exec,
        "step": {"model_flops": flops_model, "achieved_TFLOPs": round(step_tf, 1),
                 "frac": round(step_tf / MFMA_BF16_PEAK_TFLOPS, 4),
                 "note": "the reference's three products 3*2*N*H*V over the step time"},
        "dweight": {"kernel_ms": round(dw_ms, 4), "executed_flops": dw_exec,
                    "achieved_TFLOPs": round(dw_exec / (dw_ms * 1e-3) / 1e12, 1),
                    "active_tiles_bound": act_tiles},
        "fwd_obar_blocks": need_blocks,
        "kernels_ms": {k: round(v[0], 4) for k, v in kstats.items()},
    }


SAMPLE_ROWS = 256
SAMPLE_VARIANTS = {"default": dict(temperature=1.0, top_k=0, top_p=1.0, do_sample=True),
                   "default_without_log_q": dict(temperature=1.0, top_k=0, top_p=1.0,
                                                 do_sample=True, sampling_logprobs=False),
                   "topk50_topp0.9_T0.7": dict(temperature=0.7, top_k=50, top_p=0.9,
                                               do_sample=True),
                   "greedy": dict(temperature=1.0, top_k=0, top_p=1.0, do_sample=False),
                   # longer top-k lists: 65-1024 entries, and a gather past 1024
                   "topk200_T1": dict(temperature=1.0, top_k=200, top_p=1.0, do_sample=True),
                   "topk700_topp0.9": dict(temperature=1.0, top_k=700, top_p=0.9,
                                           do_sample=True),
                   # the nucleus alone (counts per key in registers, then a fill-in launch)
                   "topp0.9": dict(temperature=1.0, top_k=0, top_p=0.9, do_sample=True)}


def bench_sample(args, steps, warmup, with_cpu):
    """Rollout sampling: tokens/s of sample_next_token_batch over 256 rows of
    151936 bf16 logits (config 2's distribution), one call per step."""

    import torch

    from oracle import sampler_oracle as so
    from rosellm_amd.roseinfer import sample_next_token_batch

    device = torch.device("cuda", 0)
    B, V = SAMPLE_ROWS, 151936
    g = torch.Generator(device=device).manual_seed(args.seed)
    x = torch.randn(B, V, dtype=torch.bfloat16, device=device, generator=g).mul_(3.0)
    hot = torch.randint(0, V, (B,), device=device, generator=g)
    rows = torch.arange(0, B, 20, device=device)
    x[rows, hot[rows]] = (x[rows, hot[rows]].float() + 15.0).to(torch.bfloat16)
    from rosellm_amd import _native as nat

    def kernel_ms(kw):
        """Mean duration of `steps` launches of the entry point with the
        arguments the API passes, back to back on the stream.  The API call
        ends in a host synchronisation (its bad-row check), so an event pair
        around it would also count the launch's own submission gap on an idle
        GPU: several microseconds on a kernel of twenty."""

        tok = torch.empty(B, dtype=torch.int64, device=device)
        lp = torch.empty(B, dtype=torch.float32, device=device)
        lq = torch.empty(B, dtype=torch.float32, device=device)
        want_q = kw.get("sampling_logprobs", True)
        greedy = not kw["do_sample"] or kw["temperature"] <= 0.0

        def launch(off):
            nat.call("rrl_sample_logprobs", x.data_ptr(), nat.dtype_code(x.dtype), B, V,
                     x.stride(0), float(kw["temperature"]), int(kw["top_k"]),
                     float(kw["top_p"]), int(not greedy), args.seed, off, tok.data_ptr(),
                     lp.data_ptr(), lq.data_ptr() if want_q else None, None,
                     nat.stream_ptr(device))

        for i in range(warmup):
            launch(i)
        torch.cuda.synchronize()
        timed = nat.time_calls("rrl_sample_logprobs", capacity=steps)
        for i in range(steps):
            launch(100 + i)
        torch.cuda.synchronize()
        nat.time_calls()
        kms = [s.elapsed_time(e) for s, e in timed["rrl_sample_logprobs"]]
        return sum(kms) / len(kms)

    results = {}
    for name, kw in SAMPLE_VARIANTS.items():
        for i in range(warmup):
            sample_next_token_batch(x, seed=args.seed, offset=i, **kw)
        offs = iter(range(100, 100 + 2 * steps))
        res = timed_steps(lambda: sample_next_token_batch(x, seed=args.seed, offset=next(offs),
                                                          **kw),
                          steps, [])
        kms = [kernel_ms(kw)]
        ms = res["wall_s"] * 1e3 / steps
        results[name] = dict(ms=ms, median=statistics.median(res["step_ms"]),
                             kernel_ms=sum(kms) / len(kms))
        log(f"[bench] sample {name}: {ms:.4f} ms/step, kernel {results[name]['kernel_ms']:.4f} ms")
    head = results["default"]
    alg = B * (V * 2 + 8 + 4 + 4)  # one read of the logits; token + two log-probs out
    achieved = alg / (head["kernel_ms"] * 1e-3) / 1e9
    cpu = None
    if with_cpu:
        n = 16
        xc = x[:n].float().cpu().numpy()
        med, _ = _median_runs(lambda: so.sample_rows(xc, temperature=1.0, top_k=0, top_p=1.0,
                                                     do_sample=True, seed=args.seed, offset=0),
                              args.cpu_runs, "sampler")
        cpu = {"value": round(n / med, 1), "unit": "tokens/s", "cores": 1, "kind": "port",
               "median_s": round(med, 4),
               "sample": f"first {n} of {B} rows, oracle inverse-CDF sampler in float64 NumPy "
                         f"(one thread), median of {args.cpu_runs} runs after 1 warm-up",
               **cpu_info()}
    return {
        "metric": "tokens/sec sampled with behaviour log-probs @151936 vocab (rollout side)",
        "value": round(B / (head["ms"] * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(head["ms"], 4),
        "ms_per_step_median": round(head["median"], 4),
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


def compact(r):
    """The fields of a configuration's result kept under the headline's variants."""

    keep = {k: r.get(k) for k in ("value", "unit", "ms_per_step", "ms_per_step_median",
                                   "steps", "dtype", "step_time")}
    keep["workload"] = r["config"]["workload"]
    rf = r["roofline"]
    keep["roofline"] = {k: rf.get(k) for k in ("bound", "kernel", "achieved", "peak", "unit",
                                                "frac", "kernel_ms", "alg_bytes_per_launch",
                                                "alg_flops_per_launch", "step", "dweight",
                                                "kernels", "other_ms_per_step", "active_rows",
                                                "kernels_ms") if k in rf}
    keep["cpu_baseline"] = r.get("cpu_baseline")
    if r.get("variants"):
        keep["variants"] = r["variants"]
    return keep


def default_steps(name, args):
    """Timed steps and warm-up of a configuration: 200 / 20 for C1 and the
    sampler (sub-millisecond, host-bound steps), else --steps / --warmup
    (default 10 / 2)."""

    if name in ("c1", "sample"):
        return max(args.steps or 0, 200), max(args.warmup or 0, 20)
    return args.steps or 10, args.warmup if args.warmup is not None else 2


def calibration_conversions(device, reps=2):
    """Kernels of known traffic for the HBM counters: ``reps`` bf16 -> float32
    conversions of 2^29 random elements, each one dispatch that reads exactly
    1 GiB and writes exactly 2 GiB.  2^29 is the largest count that torch
    converts in one launch (the float32 output's largest byte offset,
    2^31 - 4, still fits its 32-bit indexing; 2^30 elements would run as two
    launches of 2^29).  A same-dtype copy would run as a DMA blit, invisible
    to the counters, and constant data could compress in the memory fabric."""

    import torch

    n = 1 << 29
    src = torch.randn(n, dtype=torch.bfloat16, device=device)
    dst = torch.empty(n, dtype=torch.float32, device=device)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] calibration: {reps} conversions, each {n * 2} B read and {n * 4} B "
        "written in one launch")
    del src, dst


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the path "
              "shards by whole GRPO groups with one scalar all-reduce per step, which "
              "is not run here.", file=sys.stderr)
        sys.exit(2)

    import gc

    import torch

    device = torch.device("cuda", 0)
    if args.objective and args.config != "c3":
        raise SystemExit("--objective applies to config c3")
    head_name = "c3_gspo_token" if args.objective == "gspo_token" else args.config
    steps, warmup = default_steps(args.config, args)
    if args.config == "sample":
        result = bench_sample(args, steps, warmup, not args.skip_cpu)
    else:
        result = measure_config(head_name, args, device, steps, warmup, not args.skip_cpu,
                                cpu_seqs=args.cpu_sample_seqs,
                                skip_masked_variant=not args.no_variants)
    gc.collect()
    torch.cuda.empty_cache()
    if args.calibrate_copy:
        calibration_conversions(device)
    if not (args.no_variants or args.headline_only):
        variants = result.setdefault("variants", {})
        for name in VARIANTS:
            if name == head_name:
                continue
            t0 = time.perf_counter()
            try:
                v_steps, v_warm = default_steps(name, args)
                if name == "sample":
                    r = bench_sample(args, v_steps, v_warm, not args.skip_cpu)
                else:
                    # C3's two objectives and C5 also time their skip_masked_rows entry
                    r = measure_config(name, args, device, v_steps, v_warm, not args.skip_cpu,
                                       skip_masked_variant=name in ("c3", "c3_gspo_token", "c5"))
                variants[name] = compact(r)
            except Exception as e:  # recorded, never fatal to the headline
                variants[name] = {"error": f"{type(e).__name__}: {e}"[:400]}
                log(f"[bench] variant {name} failed: {variants[name]['error']}")
            variants.get(name, {})["bench_s"] = round(time.perf_counter() - t0, 1)
            gc.collect()
            torch.cuda.empty_cache()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
