"""The reference's known answers run through ``import rosellm.roserlhf`` (the
opt-in shim, installed into a scratch directory only), and the
reference-dtype option held against the reference's own 16-bit ops (MI355X)."""

from __future__ import annotations

import importlib
import sys

import pytest
import torch
import torch.nn.functional as F

import rosellm_amd
from rosellm_amd import shim
from tests._cases import CASE_IDS, CASES, run_case, shim_fns

pytestmark = pytest.mark.gpu


def _drop_rosellm_modules():
    for name in [m for m in sys.modules if m == "rosellm" or m.startswith("rosellm.")]:
        del sys.modules[name]


@pytest.fixture(scope="module")
def shim_modules(tmp_path_factory):
    saved = list(sys.path)
    _drop_rosellm_modules()
    site = shim.install(tmp_path_factory.mktemp("shim_site"))
    sys.path.append(str(site))
    R = importlib.import_module("rosellm.roserlhf")
    L = importlib.import_module("rosellm.roserlhf.losses")
    assert R.__file__.startswith(str(site))
    yield R, L
    sys.path[:] = saved
    _drop_rosellm_modules()


@pytest.mark.parametrize("case", CASES, ids=CASE_IDS)
def test_known_answer_through_the_shim(case, device, shim_modules):
    print(f"[shim known-answer] {case['id']} ({case['cite']})", flush=True)
    run_case(case, "hip", device, fns=shim_fns(*shim_modules))


def _ulps16(a, b):
    """Distance in units of the last place between two bf16 tensors of equal sign."""

    ia = a.view(torch.int16).to(torch.int32)
    ib = b.view(torch.int16).to(torch.int32)
    return (ia - ib).abs()


def test_reference_dtypes_match_the_reference_ops(device, shim_modules):
    """With the option on, bf16 logits give bf16 log-probs (losses.py:34-38:
    log_softmax in the logits dtype, then gather) and a bf16 SFT loss
    (model.py:643-649: F.cross_entropy of the logits): every value within one
    bf16 ulp of the reference's ops, nearly all equal."""

    R, _L = shim_modules
    from rosellm_amd import rosetrainer as RT

    g = torch.Generator(device=device).manual_seed(91)
    x = (torch.randn(4, 64, 32000, device=device, generator=g) * 3.0).to(torch.bfloat16)
    t = torch.randint(0, 32000, (4, 64), device=device, generator=g)
    want = F.log_softmax(x, dim=-1).gather(-1, t[..., None]).squeeze(-1)
    assert R.gather_token_logprobs(x, t).dtype == torch.float32
    try:
        rosellm_amd.set_reference_dtypes(True)
        got = R.gather_token_logprobs(x, t)
        out, lp = R.fused_policy_loss(x, t, want.float(), torch.ones(4, 64, device=device),
                                      torch.ones(4, 64, dtype=torch.bool, device=device),
                                      return_logprobs=True)
        loss = RT.causal_lm_loss(x, t)
        want_loss = F.cross_entropy(x[:, :-1].reshape(-1, 32000), t[:, 1:].reshape(-1))
    finally:
        rosellm_amd.set_reference_dtypes(False)
    assert got.dtype == torch.bfloat16 and lp.dtype == torch.bfloat16
    assert loss.dtype == torch.bfloat16 and want_loss.dtype == torch.bfloat16
    d = _ulps16(got, want)
    print(f"log-probs: {(d == 0).float().mean().item():.4f} equal, max {int(d.max())} ulp",
          flush=True)
    assert int(d.max()) <= 1 and (d == 0).float().mean().item() >= 0.99
    assert torch.equal(lp, got)
    assert int(_ulps16(loss.reshape(1), want_loss.reshape(1)).max()) <= 1
