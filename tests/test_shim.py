"""The opt-in ``rosellm`` shim (rosellm_amd/shim): installed only into a
scratch directory here, it maps ``rosellm.roserlhf`` (and ``.losses``,
``.advantages``, ``.trajectory``) onto this package, and it never stands in
for a reference ``rosellm`` that is importable too.  No kernels run here."""

from __future__ import annotations

import importlib
import sys

import pytest
import torch

import rosellm_amd
from rosellm_amd import shim


def _drop_rosellm_modules():
    for name in [m for m in sys.modules if m == "rosellm" or m.startswith("rosellm.")]:
        del sys.modules[name]


@pytest.fixture
def clean_path():
    saved = list(sys.path)
    _drop_rosellm_modules()
    yield
    sys.path[:] = saved
    _drop_rosellm_modules()


def test_shim_maps_the_reference_names(tmp_path, clean_path):
    shim.install(tmp_path)
    sys.path.append(str(tmp_path))
    R = importlib.import_module("rosellm.roserlhf")
    L = importlib.import_module("rosellm.roserlhf.losses")
    A = importlib.import_module("rosellm.roserlhf.advantages")
    T = importlib.import_module("rosellm.roserlhf.trajectory")
    import rosellm_amd.roserlhf as ours
    from rosellm_amd.roserlhf import advantages as our_a, losses as our_l, trajectory as our_t

    # the reference's public names (rosellm/roserlhf/__init__.py:31-49)
    ref_names = ["GspoPolicyLossOutput", "PolicyLossOutput", "SapoPolicyLossOutput",
                 "SaoPolicyLossOutput", "broadcast_turn_advantages", "clipped_policy_loss",
                 "discounted_returns", "direct_double_sided_mask", "gather_token_logprobs",
                 "generalized_advantage_estimation", "group_standardized_advantages",
                 "leave_one_out_advantages", "gspo_policy_loss", "gspo_token_policy_loss",
                 "sapo_policy_loss", "sao_policy_loss",
                 "skip_observation_generalized_advantage_estimation"]
    for n in ref_names:
        assert getattr(R, n) is getattr(ours, n), n
        assert n in R.__all__
    assert L.masked_mean is our_l.masked_mean
    assert L.sequence_log_ratio is our_l.sequence_log_ratio
    assert A.generalized_advantage_estimation is our_a.generalized_advantage_estimation
    assert T.Trajectory is our_t.Trajectory
    with pytest.raises(FileExistsError):
        shim.install(tmp_path)


def test_shim_never_stands_in_for_the_reference(tmp_path, clean_path):
    fake = tmp_path / "ref"
    (fake / "rosellm").mkdir(parents=True)
    (fake / "rosellm" / "__init__.py").write_text("MARKER = 'reference'\n")
    site = tmp_path / "shim"
    shim.install(site)
    # the reference earlier on the path (what enable() arranges): it wins
    sys.path[:0] = [str(fake)]
    sys.path.append(str(site))
    assert importlib.import_module("rosellm").MARKER == "reference"
    _drop_rosellm_modules()
    # the shim listed first while the reference is importable: refused
    sys.path.remove(str(site))
    sys.path.insert(0, str(site))
    with pytest.raises(ImportError, match="does not stand in"):
        importlib.import_module("rosellm")


def test_enable_appends_at_the_end(clean_path):
    entry = shim.enable()
    assert sys.path[-1] == entry
    assert shim.enable() == entry and sys.path.count(entry) == 1


def test_reference_dtype_option():
    x16 = torch.zeros(3, dtype=torch.bfloat16)
    t = torch.tensor([0.1, -2.5, 3.0])
    assert not rosellm_amd.reference_dtypes()
    from rosellm_amd._config import as_reference_dtype
    assert as_reference_dtype(t, x16) is t
    try:
        rosellm_amd.set_reference_dtypes(True)
        out = as_reference_dtype(t, x16)
        assert out.dtype == torch.bfloat16 and torch.equal(out, t.to(torch.bfloat16))
        assert as_reference_dtype(t, torch.zeros(3)) is t  # float32 logits: unchanged
    finally:
        rosellm_amd.set_reference_dtypes(False)
