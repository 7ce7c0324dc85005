"""Next-token sampling with behaviour log-probs on the device, in one call.

The reference picks the next token in ``InferenceEngine._sample_next_token_batch``
(roseinfer/engine.py:1103-1171): greedy argmax, or ``logits / temperature``
restricted to the ``top_k`` largest and/or the ``top_p`` nucleus, then
``torch.multinomial`` over ``softmax(...).clamp_min(1e-9)``.  It returns the
token only, while every rollout token needs its behaviour log-probability
(``PolicyAction.old_logprobs``, roserlhf/trajectory.py:15,27-28), which the
trainer later compares with its own recomputation (the train/inference
mismatch of docs/agentic-rl/systems.md:252-274).

``sample_next_token_batch`` runs ``rrl_sample_logprobs``: one workgroup per
row chooses the token by inverse CDF with counter-based uniforms (Philox4x32-10
of row, ``offset`` and ``seed``: reproducible, no generator state on the
device; without top-k / top-p, ``max(p, 1e-9)`` is drawn as the mixture of p
and the floor's excess ``max(1e-9 - p, 0)``, a second uniform choosing the
component) and returns, with it,

* ``logprobs``: ``log_softmax(logits / T)[token]`` over the whole row (T = 1
  when greedy), formed as the training row kernels form log-probs — at T = 1
  it is the value ``gather_token_logprobs`` recomputes;
* ``sampling_logprobs``: ``log q(token)`` of the distribution actually
  sampled (after top-k / top-p and the 1e-9 floor; 0 when greedy).

The distribution is the reference's on the float32 upcast of the logits (the
reference divides by T and normalises in the logits dtype); ties at a top-k or
top-p threshold are kept lowest index first (torch.topk leaves their order
unspecified).  When sampling, rows with NaN or +inf logits raise, as
``torch.multinomial`` does; greedy decoding returns ``torch.argmax``'s token
for them (the first NaN, else the first maximum) with a NaN log-prob.
"""

from __future__ import annotations

from typing import NamedTuple, Optional

import numpy as np
import torch
from torch import Tensor

from .. import _native as nat

__all__ = ["SampleOutput", "sample_next_token", "sample_next_token_batch"]


class SampleOutput(NamedTuple):
    token_ids: Tensor                    # [B] int64
    logprobs: Tensor                     # [B] float32, log_softmax(logits / T)[token]
    sampling_logprobs: Optional[Tensor]  # [B] float32, log q(token) of the sampled
                                         # distribution (None when not asked for)


def _draw_seed(generator: Optional[torch.Generator]) -> int:
    """A 63-bit seed from a host generator (no device sync)."""

    return int(torch.randint(0, 2 ** 63 - 1, (1,), generator=generator, dtype=torch.int64).item())


def sample_next_token_batch(
    logits: Tensor,
    temperature: float,
    top_k: int,
    top_p: float,
    do_sample: bool,
    *,
    seed: Optional[int] = None,
    offset: int = 0,
    generator: Optional[torch.Generator] = None,
    sampling_logprobs: bool = True,
) -> SampleOutput:
    """Sample one token per row of ``logits`` [B, V] with the reference's
    argument meaning (roseinfer/engine.py:1103-1171) and return its
    log-probabilities.

    ``seed`` and ``offset`` fix the uniforms (row r of a call uses counter
    (r, offset)); with ``seed=None`` a seed is drawn from ``generator`` (a CPU
    ``torch.Generator``, default: torch's global one).  A decode loop can keep
    one seed and advance ``offset`` per step.

    ``sampling_logprobs=False`` skips ``log q(token)`` (the field is None).
    The token and ``logprobs`` do not change; without top-k / top-p, log q
    needs the 1e-9 floor's total mass, one more exponential per entry.
    """

    if logits.dim() != 2:
        raise ValueError(f"logits must be 2D [B, V], got shape={tuple(logits.shape)}")
    if logits.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise TypeError("logits must be float32, bfloat16 or float16")
    dev = nat.require_device(logits)
    x = logits if logits.stride(-1) == 1 else logits.contiguous()
    B, V = x.shape
    if V == 0:
        raise ValueError("logits need at least one vocabulary entry")
    if seed is None:
        seed = _draw_seed(generator)
    tokens = torch.empty(B, dtype=torch.int64, device=dev)
    logp = torch.empty(B, dtype=torch.float32, device=dev)
    logq = torch.empty(B, dtype=torch.float32, device=dev) if sampling_logprobs else None
    # No status word: a row with NaN or +inf logits (or no finite maximum)
    # gets a NaN log-prob, and every other row a finite one, so one copy of
    # the log-probs to the host (the synchronisation the reference's own
    # validity check makes) finds them without a separately zeroed flag.
    nat.call("rrl_sample_logprobs", x.data_ptr(), nat.dtype_code(x.dtype), B, V,
             x.stride(0) if B > 1 else V, float(temperature), int(top_k), float(top_p),
             int(bool(do_sample)), int(seed) & (2 ** 64 - 1), int(offset) & (2 ** 64 - 1),
             tokens.data_ptr(), logp.data_ptr(), logq.data_ptr() if logq is not None else None,
             None, nat.stream_ptr(dev))
    # Sampling raises on such rows, as torch.multinomial does; NaN anywhere
    # makes the sum NaN (the log-probs are never +inf).  Greedy decoding is
    # torch.argmax in the reference (engine.py:1117-1118), which never raises:
    # its bad rows keep their argmax token (NaN ranking above every number)
    # and a NaN log-prob, and the call makes no host synchronisation.
    greedy = (not do_sample) or temperature <= 0.0
    if B and not greedy and bool(np.isnan(logp.cpu().numpy().sum())):
        raise RuntimeError("probability tensor contains either `inf`, `nan` or element < 0")
    return SampleOutput(tokens, logp, logq)


def sample_next_token(logits: Tensor, temperature: float, top_k: int, top_p: float,
                      do_sample: bool, **kw) -> int:
    """The single-sequence form (roseinfer/engine.py:1088-1101): ``logits``
    [..., V] are viewed as rows and the first row's token is returned."""

    rows = logits.reshape(-1, int(logits.size(-1)))
    return int(sample_next_token_batch(rows, temperature, top_k, top_p, do_sample,
                                       **kw).token_ids[0].item())
