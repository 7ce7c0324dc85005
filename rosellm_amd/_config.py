"""Process-wide options of rosellm_amd.

``reference_dtypes``: the reference returns token log-probabilities
(rosellm/roserlhf/losses.py:34-38, ``log_softmax`` in the logits dtype) and the
SFT loss (rosetrainer/model.py:643-649, ``F.cross_entropy`` of the logits) in
the logits' own dtype; this package returns them in float32 (float64 for
float64 logits).  With the option on, 16-bit logits give 16-bit log-probs and
losses: the float32 results rounded once to the logits dtype (round to
nearest even), which is what the reference's 16-bit ops store after computing
in float32.  Off by default; on when the environment variable
``ROSELLM_AMD_REFERENCE_DTYPES`` is set to anything but ``0`` or empty, or
after ``set_reference_dtypes(True)``.
"""

from __future__ import annotations

import os

_state = {"reference_dtypes": os.environ.get("ROSELLM_AMD_REFERENCE_DTYPES", "") not in ("", "0")}


def reference_dtypes() -> bool:
    """Whether log-probs and losses come back in the logits dtype."""

    return _state["reference_dtypes"]


def set_reference_dtypes(on: bool) -> None:
    """Turn the reference-dtype results on or off for this process."""

    _state["reference_dtypes"] = bool(on)


def as_reference_dtype(t, like):
    """``t`` in ``like``'s dtype when the option is on and ``like`` is 16-bit,
    else ``t`` unchanged (differentiable)."""

    import torch

    if _state["reference_dtypes"] and like.dtype in (torch.bfloat16, torch.float16):
        return t.to(like.dtype)
    return t
