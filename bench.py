#!/usr/bin/env python3
"""Throughput of the RoseRLHF GRPO training-step hot path on one MI355X.

Workload: 32 prompts x group 8 = 256 sequences x 1024
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
    # name: (prompts, group, T, V, logits dtype, sigma, hot fraction, old-logp noise,
    #        length range, clip_low, clip_high)
    "c2": dict(prompts=32, group=8, T=1024, V=151936, dtype="bfloat16", sigma=3.0, hot=0.05,
               noise=0.1, lengths=(64, 1024), clip_low=0.2, clip_high=0.28,
               workload="C2: GRPO token-level PPO-clip fwd+bwd, 256x1024 tokens, V=151936 bf16"),
    "c1": dict(prompts=8, group=4, T=128, V=50257, dtype="float32", sigma=2.0, hot=0.0,
               noise=0.05, lengths=(16, 128), clip_low=0.2, clip_high=None,
               workload="C1: GRPO token-level PPO-clip fwd+bwd, 32x128 tokens, V=50257 fp32"),
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=2)
    p.add_argument("--config", choices=sorted(CONFIGS), default="c2")
    p.add_argument("--path", choices=["fused", "composed"], default="fused")
    p.add_argument("--cpu-sample-seqs", type=int, default=2,
                   help="sequences of the batch timed on the CPU oracle")
    p.add_argument("--cpu-runs", type=int, default=3)
    p.add_argument("--skip-cpu", action="store_true")
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
    gens = [torch.Generator(device=device).manual_seed(seed + i) for i in range(8)]
    logits = torch.randn(B, T, V, dtype=dtype, device=device, generator=gens[0])
    logits.mul_(cfg["sigma"])
    flat = logits.view(-1, V)
    if cfg["hot"] > 0:
        hot_rows = torch.nonzero(torch.rand(B * T, device=device, generator=gens[1]) < cfg["hot"])
        hot_rows = hot_rows.reshape(-1)
        hot_cols = torch.randint(0, V, (hot_rows.numel(),), device=device, generator=gens[2])
        flat[hot_rows, hot_cols] = (flat[hot_rows, hot_cols].float() + 15.0).to(dtype)
    # Actions ~ softmax(logits) by Gumbel-max; reference log-probs by
    # log_softmax in float32, chunked so no [N, V] float32 tensor is built.
    actions = torch.empty(B * T, dtype=torch.int64, device=device)
    logp = torch.empty(B * T, dtype=torch.float32, device=device)
    chunk = max(1, (1 << 30) // (V * 4))
    for r0 in range(0, B * T, chunk):
        xf = flat[r0:r0 + chunk].float()
        u = torch.rand(xf.shape, device=device, generator=gens[3]).clamp_(min=1e-20)
        a = torch.argmax(xf - torch.log(-torch.log(u)), dim=-1)
        actions[r0:r0 + chunk] = a
        logp[r0:r0 + chunk] = torch.log_softmax(xf, dim=-1).gather(1, a[:, None]).squeeze(1)
        del xf, u
    actions = actions.view(B, T)
    old = (logp + cfg["noise"] * torch.randn(B * T, device=device, generator=gens[4])).view(B, T)
    rewards = torch.randint(0, 2, (cfg["prompts"], cfg["group"]), device=device,
                            generator=gens[5]).float()
    lo, hi = cfg["lengths"]
    lengths = torch.randint(lo, hi + 1, (B,), device=device, generator=gens[6])
    mask = torch.arange(T, device=device)[None, :] < lengths[:, None]
    return dict(logits=logits, actions=actions, old=old, rewards=rewards, mask=mask, B=B, T=T,
                V=V)


def make_step(inp, cfg, path):
    import torch

    from rosellm_amd import roserlhf as R

    logits = inp["logits"].requires_grad_()
    actions, old, rewards, mask = inp["actions"], inp["old"], inp["rewards"], inp["mask"]
    B, T = inp["B"], inp["T"]
    kw = dict(clip_low=cfg["clip_low"], clip_high=cfg["clip_high"])

    def advantages():
        seq = R.group_standardized_advantages(rewards).reshape(-1)
        return seq[:, None].expand(B, T)

    if path == "fused":
        def step():
            logits.grad = None
            out = R.fused_policy_loss(logits, actions, old, advantages(), mask, **kw)
            out.loss.backward()
            return out
    else:
        def step():
            logits.grad = None
            lp = R.gather_token_logprobs(logits, actions)
            out = R.clipped_policy_loss(lp, old, advantages(), mask, **kw)
            out.loss.backward()
            return out
    return step


def cpu_baseline(inp, cfg, n_seq, runs):
    """The oracle's PyTorch-CPU composition (log_softmax -> gather -> clip ->
    autograd), op for op the reference's, timed on the first n_seq sequences."""

    import torch

    from oracle import roserlhf_oracle as o

    T = inp["T"]
    x = inp["logits"].detach()[:n_seq].cpu()
    t = inp["actions"][:n_seq].cpu()
    old = inp["old"][:n_seq].cpu()
    mask = inp["mask"][:n_seq].cpu()
    seq_adv = o.group_standardize(inp["rewards"].cpu()).reshape(-1)[:n_seq]
    adv = seq_adv[:, None].expand(n_seq, T)
    threads = torch.get_num_threads()
    times = []
    for i in range(runs + 1):
        t0 = time.perf_counter()
        o.grpo_step(x, t, old, adv, mask, clip_low=cfg["clip_low"], clip_high=cfg["clip_high"])
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
                   f"tensors), oracle log_softmax->gather->clip->autograd on the fp32 upcast, "
                   f"median of {runs} runs after 1 warm-up, torch threads={threads}, "
                   f"os.cpu_count()={os.cpu_count()}"),
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


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the path "
              "shards by whole GRPO groups with one scalar all-reduce (see DESIGN.md), which "
              "is not run here.", file=sys.stderr)
        sys.exit(2)

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
    step = make_step(inp, cfg, args.path)

    for i in range(args.warmup):
        step()
        torch.cuda.synchronize()
        log(f"[bench] warmup {i} done")

    kernel = "rrl_fused_logprob_policy" if args.path == "fused" else "rrl_logprob_bwd"
    timed = nat.time_calls(kernel)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    nat.time_calls()
    ms_step = elapsed * 1e3 / args.steps
    tok_s = N / (elapsed / args.steps)
    kms = [s.elapsed_time(e) for s, e in timed[kernel]]
    k_avg = sum(kms) / len(kms)
    log(f"[bench] {args.steps} steps: {ms_step:.3f} ms/step, {tok_s / 1e6:.3f} M tok/s; "
        f"{kernel} avg {k_avg:.3f} ms over {len(kms)} launches; loss {out.loss.item():.6g}")

    in_b = inp["logits"].element_size()
    alg_bytes = N * (V * (in_b + in_b) + SIDE_BYTES)
    if args.path == "composed":
        # the backward sweep alone: read logits, write dlogits, plus its row scalars
        alg_bytes = N * (V * (in_b + in_b) + 8 + 4 + 4 + 4)
    achieved = alg_bytes / (k_avg * 1e-3) / 1e9
    workload_key = f"{args.config}-{args.path}"
    roofline = {
        "bound": "hbm",
        "kernel": kernel,
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic_from_profiles(kernel, workload_key),
        "kernel_ms": round(k_avg, 4),
        "alg_bytes_per_launch": alg_bytes,
    }

    if args.calibrate_copy:
        # 4 GiB device-to-device copy: FETCH_SIZE / WRITE_SIZE of this kernel
        # give the counters' bytes-per-unit scale.
        src = torch.empty(1 << 31, dtype=torch.int16, device=device).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] calibration copy: {src.numel() * 2} bytes read and written")
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
            "path": args.path,
            "sequences": inp["B"],
            "seq_len": inp["T"],
            "vocab": V,
            "tokens_per_step": N,
            "parallelism": "none (1 GPU)",
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
