"""Run the transcribed reference known answers (tests/golden/known_answers.json)
against either the CPU oracle or the HIP-backed package."""

from __future__ import annotations

import json
import math
from pathlib import Path
from typing import Any, Dict

import pytest
import torch

GOLDEN = Path(__file__).resolve().parent / "golden" / "known_answers.json"


def load_cases():
    return json.loads(GOLDEN.read_text())["cases"]


def _oracle_fns():
    from oracle import roserlhf_oracle as o

    def gspo_adv(cur, roll, adv, mask, **kw):
        return o.gspo(cur, roll, adv, mask, **kw)

    return {
        "gather_token_logprobs": lambda logits, target_ids: o.token_logprobs(logits, target_ids),
        "clipped_policy_loss": o.ppo_clip,
        "sequence_log_ratio": o.sequence_log_ratio,
        "direct_double_sided_mask": o.strict_trust,
        "sao_policy_loss": o.sao,
        "gspo_policy_loss": gspo_adv,
        "gspo_token_policy_loss": o.gspo_token,
        "sapo_policy_loss": o.sapo,
        "discounted_returns": o.returns_to_go,
        "generalized_advantage_estimation": o.gae,
        "leave_one_out_advantages": o.leave_one_out,
        "group_standardized_advantages": o.group_standardize,
        "broadcast_turn_advantages": o.turn_broadcast,
        "skip_observation_generalized_advantage_estimation": o.skip_observation_gae,
    }


def _hip_fns():
    from rosellm_amd import roserlhf as r
    from rosellm_amd.roserlhf import losses as L

    names = [
        "gather_token_logprobs", "clipped_policy_loss", "direct_double_sided_mask",
        "sao_policy_loss", "gspo_policy_loss", "gspo_token_policy_loss", "sapo_policy_loss",
        "discounted_returns", "generalized_advantage_estimation", "leave_one_out_advantages",
        "group_standardized_advantages", "broadcast_turn_advantages",
        "skip_observation_generalized_advantage_estimation",
    ]
    fns = {n: getattr(r, n) for n in names}
    fns["sequence_log_ratio"] = L.sequence_log_ratio
    return fns


def _tensor(v, dtype: torch.dtype, device) -> torch.Tensor:
    def flat(x):
        return [y for z in x for y in flat(z)] if isinstance(x, list) else [x]

    vals = flat(v)
    if vals and all(isinstance(x, bool) for x in vals):
        return torch.tensor(v, dtype=torch.bool, device=device)
    if vals and all(isinstance(x, int) and not isinstance(x, bool) for x in vals):
        return torch.tensor(v, dtype=torch.int64, device=device)
    return torch.tensor(v, dtype=dtype, device=device)


def _field(out: Any, name: str):
    if name == "out":
        return out
    if name in ("out0", "out1"):
        return out[int(name[-1])]
    if isinstance(out, dict):
        return out[name]
    return getattr(out, name)


def shim_fns(R, L):
    """The same functions taken from a ``rosellm.roserlhf`` package (the
    opt-in shim) and its ``losses`` module."""

    names = [
        "gather_token_logprobs", "clipped_policy_loss", "direct_double_sided_mask",
        "sao_policy_loss", "gspo_policy_loss", "gspo_token_policy_loss", "sapo_policy_loss",
        "discounted_returns", "generalized_advantage_estimation", "leave_one_out_advantages",
        "group_standardized_advantages", "broadcast_turn_advantages",
        "skip_observation_generalized_advantage_estimation",
    ]
    fns = {n: getattr(R, n) for n in names}
    fns["sequence_log_ratio"] = L.sequence_log_ratio
    return fns


def run_case(case: Dict[str, Any], backend: str, device, fns=None) -> None:
    if fns is None:
        fns = _oracle_fns() if backend == "oracle" else _hip_fns()
    fn = fns[case["fn"]]
    dtype = getattr(torch, case["dtype"])
    args = {k: _tensor(v, dtype, device) for k, v in case["args"].items()}
    for name in case["grad"]:
        args[name].requires_grad_(True)
    kwargs = dict(case["kwargs"])
    for k, v in case["tensor_kwargs"].items():
        kwargs[k] = _tensor(v, dtype, device)
    if case["raises"]:
        exc = {"ValueError": ValueError, "TypeError": TypeError}[case["raises"]["type"]]
        with pytest.raises(exc, match=case["raises"]["match"]):
            fn(*args.values(), **kwargs)
        return
    out = fn(*args.values(), **kwargs)
    tol = case.get("tol")
    for name, want in case["expect"].items():
        got = _field(out, name)
        if isinstance(want, list) or (isinstance(got, torch.Tensor) and got.dim() > 0):
            w = _tensor(want, got.dtype if got.is_floating_point() else dtype, "cpu")
            if w.dtype == torch.bool:
                assert torch.equal(got.cpu(), w), (case["id"], name, got, w)
            else:
                kw = {} if tol is None else {"rtol": 0.0, "atol": tol}
                torch.testing.assert_close(got.detach().cpu().to(w.dtype), w, **kw,
                                           msg=f"{case['id']}:{name}")
        else:
            g = float(got.detach().cpu())
            if tol is None:
                assert g == pytest.approx(want, rel=1e-6, abs=1e-6), (case["id"], name, g, want)
            else:
                assert abs(g - want) <= tol + 1e-12, (case["id"], name, g, want)
    if case["grad"]:
        _field(out, case["grad_of"]).backward()
        for name, want in case["grad"].items():
            got = args[name].grad
            if want is None:
                assert got is None, (case["id"], name, got)
                continue
            assert got is not None, (case["id"], name)
            w = torch.tensor(want, dtype=got.dtype)
            torch.testing.assert_close(got.cpu(), w, msg=f"{case['id']}:grad {name}")
            # a masked gradient is exactly zero, not merely small
            for gv, wv in zip(got.cpu().reshape(-1).tolist(), w.reshape(-1).tolist()):
                if wv == 0.0:
                    assert gv == 0.0, (case["id"], name, gv)


CASES = load_cases()
CASE_IDS = [c["id"] for c in CASES]
