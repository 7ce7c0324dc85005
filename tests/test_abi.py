"""The C ABI library without a GPU: it loads, exports every entry point that
include/roserlhf_amd.h declares, and its host-side validation returns the
documented status codes before any device work.  Also the Python API's
argument validation, which runs before any tensor reaches a device."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from rosellm_amd import _native as nat

HEADER = Path(__file__).resolve().parents[1] / "include" / "roserlhf_amd.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"RRL_API\s+[\w\s\*]+?\b(rrl_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not nat.LIB_PATH.exists():
        pytest.skip("librosellm_amd.so is not built (run __graft_entry__.build())")
    return nat.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = declared_functions()
    assert len(names) >= 20, names
    for n in names:
        assert hasattr(lib, n), f"{n} declared in the header but not exported"
    assert set(names) == set(nat.SIGNATURES), (
        "ctypes signatures and header declarations differ: "
        f"{sorted(set(names) ^ set(nat.SIGNATURES))}")


def test_abi_version_matches_header(lib):
    want = int(re.search(r"#define RRL_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert lib.rrl_abi_version() == want


def test_workspace_size_queries(lib):
    assert lib.rrl_policy_workspace_bytes(256, nat.F32) >= 256 * 9 * 4
    assert lib.rrl_policy_workspace_bytes(256, nat.F64) >= 256 * 9 * 8
    assert lib.rrl_fused_records_bytes(256, 1024) >= 256 * 1024 * 16
    assert lib.rrl_reduce_workspace_bytes(1000) > 0


def test_host_validation_status_codes(lib):
    tv = nat.RrlView(None, nat.I64, 1, 1)
    # a non-float logits dtype is rejected before any launch
    rc = lib.rrl_logprob_fwd(None, nat.I32, 2, 3, 10, 30, 10, tv, None, nat.F32, None, None,
                             None)
    assert rc == -2 and b"float" in lib.rrl_last_error()
    # negative sizes
    rc = lib.rrl_logprob_fwd(None, nat.F32, -1, 3, 10, 30, 10, tv, None, nat.F32, None, None,
                             None)
    assert rc == -1
    # an unknown objective kind
    p = nat.RrlPolicyParams(99, 0, 0, 0, 0.2, 0.2, 20.0, 1.0, 1.0)
    nv = nat.NONE_VIEW
    rc = lib.rrl_policy_fwd(ctypes.byref(p), 1, 1, nv, nv, nv, nv, nat.F32, None, None, None,
                            None, None, None)
    assert rc == -1 and b"objective" in lib.rrl_last_error()
    # the single pass accepts only the token-local objectives
    p = nat.RrlPolicyParams(nat.OBJ_GSPO, 0, 0, 0, 0.2, 0.2, 20.0, 1.0, 1.0)
    rc = lib.rrl_fused_logprob_policy(ctypes.byref(p), None, nat.BF16, 1, 1, 8, 8, 8, tv, nv,
                                      nv, nv, None, None, None, None, None, nat.BF16, 8, 8,
                                      None, None)
    assert rc == -1 and b"token-local" in lib.rrl_last_error()
    # the weight transpose: negative sizes, null operands, short row strides
    rc = lib.rrl_transpose16(None, -1, 4, 4, None, 4, None)
    assert rc == -1 and b"negative" in lib.rrl_last_error()
    assert lib.rrl_transpose16(None, 0, 4, 4, None, 0, None) == 0  # nothing to do
    rc = lib.rrl_transpose16(None, 4, 4, 4, None, 4, None)
    assert rc == -1 and b"null" in lib.rrl_last_error()
    rc = lib.rrl_transpose16(16, 4, 8, 4, 16, 4, None)
    assert rc == -1 and b"stride" in lib.rrl_last_error()
    rc = lib.rrl_transpose16(16, 4, 8, 8, 16, 2, None)
    assert rc == -1 and b"stride" in lib.rrl_last_error()
    # the sampler: logits dtype and row count
    rc = lib.rrl_sample_logprobs(16, nat.I32, 1, 8, 8, 1.0, 0, 1.0, 1, 0, 0, 16, 16, None, None,
                                 None)
    assert rc == -2 and b"float32, bfloat16 or float16" in lib.rrl_last_error()
    rc = lib.rrl_sample_logprobs(16, nat.BF16, -1, 8, 8, 1.0, 0, 1.0, 1, 0, 0, 16, 16, None,
                                 None, None)
    assert rc == -1 and b"rows" in lib.rrl_last_error()
    # success clears the last error
    assert lib.rrl_abi_version() >= 1


# ---- Python API validation (reference messages; no device needed) ----------


def test_api_validation_matches_reference_messages():
    from rosellm_amd import roserlhf as R
    from rosellm_amd.roserlhf import losses as L

    z = torch.zeros(2, 3)
    with pytest.raises(ValueError, match="logits must include positions"):
        R.gather_token_logprobs(torch.zeros(5), torch.zeros((), dtype=torch.long))
    with pytest.raises(ValueError, match="must match logits prefix"):
        R.gather_token_logprobs(torch.zeros(2, 3, 7), torch.zeros(2, 4, dtype=torch.long))
    with pytest.raises(TypeError, match="integer tensor"):
        R.gather_token_logprobs(torch.zeros(2, 3, 7), torch.zeros(2, 3))
    with pytest.raises(ValueError, match="same shape"):
        R.clipped_policy_loss(z, z, z, torch.zeros(2, 4, dtype=torch.bool))
    with pytest.raises(ValueError, match="clip_low must be non-negative"):
        R.clipped_policy_loss(z, z, z, z.bool(), clip_low=-0.1)
    with pytest.raises(ValueError, match="max_log_ratio must exceed"):
        R.sao_policy_loss(z, z, z, z.bool(), clip_low=0.2, clip_high=0.2, max_log_ratio=0.1)
    with pytest.raises(ValueError, match="rank-2"):
        R.gspo_policy_loss(torch.zeros(2, 3, 4), torch.zeros(2, 3, 4), torch.zeros(2, 3),
                           torch.zeros(2, 3, 4).bool(), clip_low=0.1, clip_high=0.1)
    with pytest.raises(ValueError, match="sequence_advantages must have shape"):
        R.gspo_policy_loss(z, z, torch.zeros(3), z.bool(), clip_low=0.1, clip_high=0.1)
    with pytest.raises(ValueError, match="temperatures must be positive"):
        R.sapo_policy_loss(z, z, z, z.bool(), tau_positive=0.0)
    with pytest.raises(ValueError, match="group_size"):
        R.group_standardized_advantages(torch.zeros(3, 1))
    with pytest.raises(ValueError, match="group_size"):
        R.leave_one_out_advantages(torch.zeros(3, 1))
    with pytest.raises(ValueError, match="gamma must be in"):
        R.discounted_returns(z, gamma=1.5)
    with pytest.raises(ValueError, match="gae_lambda must be in"):
        R.generalized_advantage_estimation(z, z, gae_lambda=-0.5)
    with pytest.raises(ValueError, match="turn_advantages must have shape"):
        R.broadcast_turn_advantages(torch.zeros(3), torch.zeros(2, 3, dtype=torch.long),
                                    z.bool())
    with pytest.raises(ValueError, match="values and mask must have the same shape"):
        L.masked_mean(z, torch.zeros(3, 2))
    with pytest.raises(ValueError, match="rank-2"):
        L.sequence_log_ratio(torch.zeros(2, 3, 4), torch.zeros(2, 3, 4), torch.zeros(2, 3, 4))


def test_api_has_no_cpu_fallback():
    """Valid CPU tensors reach the device check and raise: the product path
    never computes on the host."""

    from rosellm_amd import roserlhf as R

    z = torch.zeros(2, 3)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        R.clipped_policy_loss(z, z, z, z.bool())
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        R.gather_token_logprobs(torch.zeros(2, 3, 7), torch.zeros(2, 3, dtype=torch.long))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        R.group_standardized_advantages(torch.zeros(4, 8))
