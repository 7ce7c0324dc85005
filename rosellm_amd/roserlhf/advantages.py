"""Advantage estimators on MI355X (drop-in for ``rosellm/roserlhf/advantages.py``).

The final axis is time or group unless a function says otherwise.  Reverse
recurrences run as per-sequence segmented affine scans in one HIP launch (the
reference walks time in a Python loop, about ten ATen dispatches per step);
group statistics, leave-one-out and turn broadcasting are single launches.
Inputs must be ROCm device tensors; there is no CPU path.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from .. import _native as nat

__all__ = [
    "broadcast_turn_advantages",
    "discounted_returns",
    "generalized_advantage_estimation",
    "group_standardized_advantages",
    "leave_one_out_advantages",
    "masked_whiten",
    "skip_observation_generalized_advantage_estimation",
]


def _as_bool_mask(mask: Optional[Tensor], like: Tensor) -> Optional[Tensor]:
    """advantages.py:17-22: None means all-true; shape must match; nonzero is true.

    Returns None for "no mask" so the kernel treats every step as set.
    """

    if mask is None:
        return None
    if mask.shape != like.shape:
        raise ValueError(f"mask shape {mask.shape} must match {like.shape}")
    return mask if mask.device == like.device else mask.to(like.device)


def _time_view(t: Optional[Tensor], B: int, T: int):
    if t is None:
        return nat.NONE_VIEW, None
    return nat.rows_view(t, B, T)


def _bootstrap_view(bootstrap: Optional[Tensor], batch_shape, like: Tensor):
    if bootstrap is None:
        return nat.NONE_VIEW, None
    if bootstrap.shape != batch_shape:
        raise ValueError(f"bootstrap_value shape {bootstrap.shape} must be {batch_shape}")
    b = bootstrap if bootstrap.device == like.device else bootstrap.to(like.device)
    return nat.vector_view(b)


def discounted_returns(
    rewards: Tensor,
    *,
    gamma: float = 1.0,
    terminated: Optional[Tensor] = None,
    valid_mask: Optional[Tensor] = None,
    bootstrap_value: Optional[Tensor] = None,
) -> Tensor:
    """Reward-to-go on the final dimension (advantages.py:25-80).

    ``terminated`` cuts the future at a true terminal; a time-limit truncation
    is a final valid step with ``terminated=False`` and a ``bootstrap_value``;
    padded (``valid_mask=False``) steps neither add reward nor propagate return.
    """

    if rewards.ndim < 1:
        raise ValueError("rewards must have a time dimension")
    if not rewards.is_floating_point():
        raise TypeError("rewards must be floating point")
    if not 0.0 <= gamma <= 1.0:
        raise ValueError("gamma must be in [0, 1]")
    valid = _as_bool_mask(valid_mask, rewards)
    terminal = _as_bool_mask(terminated, rewards)
    batch_shape = rewards.shape[:-1]
    dev = nat.require_device(rewards)
    B, T = nat.flatten_rows(rewards.shape)
    rv, _rk = nat.rows_view(rewards, B, T)
    tv, _tk = _time_view(terminal, B, T)
    vv, _vk = _time_view(valid, B, T)
    bv, _bk = _bootstrap_view(bootstrap_value, batch_shape, rewards)
    acc = nat.acc_dtype(rewards.dtype)
    out = torch.empty(rewards.shape, dtype=acc, device=dev)
    nat.call("rrl_discounted_returns", B, T, rv, tv, vv, bv, float(gamma), out.data_ptr(),
             nat.dtype_code(acc), nat.stream_ptr(dev))
    return out.to(rewards.dtype)


def generalized_advantage_estimation(
    rewards: Tensor,
    values: Tensor,
    *,
    gamma: float = 1.0,
    gae_lambda: float = 1.0,
    terminated: Optional[Tensor] = None,
    valid_mask: Optional[Tensor] = None,
    bootstrap_value: Optional[Tensor] = None,
) -> Tuple[Tensor, Tensor]:
    """GAE advantages and value targets (advantages.py:83-142).

    True terminals cut both the TD bootstrap and the trace; padding is skipped
    (the next valid value and trace carry across it).
    """

    if rewards.shape != values.shape:
        raise ValueError("rewards and values must have the same shape")
    if not rewards.is_floating_point() or not values.is_floating_point():
        raise TypeError("rewards and values must be floating point")
    if not 0.0 <= gamma <= 1.0:
        raise ValueError("gamma must be in [0, 1]")
    if not 0.0 <= gae_lambda <= 1.0:
        raise ValueError("gae_lambda must be in [0, 1]")
    valid = _as_bool_mask(valid_mask, rewards)
    terminal = _as_bool_mask(terminated, rewards)
    batch_shape = rewards.shape[:-1]
    dev = nat.require_device(rewards, values)
    B, T = nat.flatten_rows(rewards.shape)
    rv, _rk = nat.rows_view(rewards, B, T)
    valv, _valk = nat.rows_view(values, B, T)
    tv, _tk = _time_view(terminal, B, T)
    vv, _vk = _time_view(valid, B, T)
    bv, _bk = _bootstrap_view(bootstrap_value, batch_shape, rewards)
    acc = nat.acc_dtype(rewards.dtype, values.dtype)
    adv = torch.empty(rewards.shape, dtype=acc, device=dev)
    tgt = torch.empty(rewards.shape, dtype=acc, device=dev)
    nat.call("rrl_gae", B, T, rv, valv, tv, vv, bv, float(gamma), float(gae_lambda),
             adv.data_ptr(), tgt.data_ptr(), nat.dtype_code(acc), nat.stream_ptr(dev))
    return adv.to(rewards.dtype), tgt.to(torch.promote_types(rewards.dtype, values.dtype))


def skip_observation_generalized_advantage_estimation(
    rewards: Tensor,
    action_end_values: Tensor,
    next_action_values: Tensor,
    *,
    gamma: float = 1.0,
    gae_lambda: float = 1.0,
    terminated: Optional[Tensor] = None,
    valid_mask: Optional[Tensor] = None,
) -> Tuple[Tensor, Tensor]:
    """SAO's action-to-action GAE across environment observations
    (advantages.py:145-217); one position per semantic model action."""

    if not (rewards.shape == action_end_values.shape == next_action_values.shape):
        raise ValueError("rewards and action-value tensors must have the same shape")
    if rewards.ndim < 1:
        raise ValueError("inputs must have an action-time dimension")
    if not (
        rewards.is_floating_point()
        and action_end_values.is_floating_point()
        and next_action_values.is_floating_point()
    ):
        raise TypeError("rewards and values must be floating point")
    if not 0.0 <= gamma <= 1.0:
        raise ValueError("gamma must be in [0, 1]")
    if not 0.0 <= gae_lambda <= 1.0:
        raise ValueError("gae_lambda must be in [0, 1]")
    valid = _as_bool_mask(valid_mask, rewards)
    terminal = _as_bool_mask(terminated, rewards)
    dev = nat.require_device(rewards, action_end_values, next_action_values)
    B, T = nat.flatten_rows(rewards.shape)
    rv, _rk = nat.rows_view(rewards, B, T)
    ev, _ek = nat.rows_view(action_end_values, B, T)
    nv, _nk = nat.rows_view(next_action_values, B, T)
    tv, _tk = _time_view(terminal, B, T)
    vv, _vk = _time_view(valid, B, T)
    acc = nat.acc_dtype(rewards.dtype, action_end_values.dtype, next_action_values.dtype)
    adv = torch.empty(rewards.shape, dtype=acc, device=dev)
    tgt = torch.empty(rewards.shape, dtype=acc, device=dev)
    nat.call("rrl_skip_observation_gae", B, T, rv, ev, nv, tv, vv, float(gamma),
             float(gae_lambda), adv.data_ptr(), tgt.data_ptr(), nat.dtype_code(acc),
             nat.stream_ptr(dev))
    return adv.to(rewards.dtype), tgt.to(torch.promote_types(rewards.dtype,
                                                             action_end_values.dtype))


def _groups_last(rewards: Tensor, dim: int):
    moved = rewards.movedim(dim, -1)
    G = moved.shape[-1]
    n = moved.numel() // G if G else 0
    view, keep = nat.rows_view(moved, n, G)
    return moved.shape, n, G, view, keep


def leave_one_out_advantages(rewards: Tensor, *, dim: int = -1) -> Tensor:
    """``r_i - mean_{k != i} r_k`` within each group (advantages.py:220-233)."""

    if not rewards.is_floating_point():
        raise TypeError("rewards must be floating point")
    group_size = rewards.shape[dim]
    if group_size < 2:
        raise ValueError("leave-one-out advantages require group_size >= 2")
    dev = nat.require_device(rewards)
    moved_shape, n, G, view, _keep = _groups_last(rewards, dim)
    acc = nat.acc_dtype(rewards.dtype)
    out = torch.empty(moved_shape, dtype=acc, device=dev)
    nat.call("rrl_leave_one_out", n, G, view, out.data_ptr(), nat.dtype_code(acc),
             nat.stream_ptr(dev))
    return out.movedim(-1, dim).to(rewards.dtype)


def group_standardized_advantages(
    rewards: Tensor,
    *,
    dim: int = -1,
    eps: float = 1e-8,
) -> Tensor:
    """Center and population-standardize within a rollout group
    (advantages.py:236-258); uniform groups return exactly zero."""

    if not rewards.is_floating_point():
        raise TypeError("rewards must be floating point")
    if rewards.shape[dim] < 2:
        raise ValueError("group standardization requires group_size >= 2")
    if eps <= 0:
        raise ValueError("eps must be positive")
    dev = nat.require_device(rewards)
    moved_shape, n, G, view, _keep = _groups_last(rewards, dim)
    acc = nat.acc_dtype(rewards.dtype)
    out = torch.empty(moved_shape, dtype=acc, device=dev)
    nat.call("rrl_group_standardize", n, G, view, float(eps), out.data_ptr(),
             nat.dtype_code(acc), nat.stream_ptr(dev))
    return out.movedim(-1, dim).to(rewards.dtype)


def broadcast_turn_advantages(
    turn_advantages: Tensor,
    turn_ids: Tensor,
    action_mask: Tensor,
) -> Tensor:
    """Map ``[batch, turns]`` advantages to policy-token positions
    (advantages.py:261-290).  Masked positions get zero whatever their id;
    an unmasked position with an out-of-range id raises."""

    if turn_advantages.ndim != 2:
        raise ValueError("turn_advantages must have shape [batch, turns]")
    if turn_ids.ndim != 2 or action_mask.ndim != 2:
        raise ValueError("turn_ids and action_mask must be rank-2")
    if turn_ids.shape != action_mask.shape:
        raise ValueError("turn_ids and action_mask must have the same shape")
    if turn_ids.shape[0] != turn_advantages.shape[0]:
        raise ValueError("batch dimensions must match")
    dev = nat.require_device(turn_advantages)
    ids = turn_ids if turn_ids.device == dev else turn_ids.to(dev)
    mask = action_mask if action_mask.device == dev else action_mask.to(dev)
    B, T = ids.shape
    K = turn_advantages.shape[1]
    av, _ak = nat.rows_view(turn_advantages, B, K)
    iv, _ik = nat.rows_view(ids, B, T)
    mv, _mk = nat.rows_view(mask, B, T)
    acc = nat.acc_dtype(turn_advantages.dtype)
    out = torch.empty((B, T), dtype=acc, device=dev)
    status = nat.new_status(dev)
    nat.call("rrl_broadcast_turn", B, K, T, av, iv, mv, out.data_ptr(), nat.dtype_code(acc),
             status.data_ptr(), nat.stream_ptr(dev))
    if B * T and nat.read_status(status) & nat.FLAG_INVALID_TURN:
        raise ValueError("an unmasked policy token has an invalid turn ID")
    return out.to(turn_advantages.dtype)


def masked_whiten(
    values: Tensor,
    mask: Tensor,
    *,
    eps: float = 1e-8,
    shift_mean: bool = True,
) -> Tensor:
    """Whiten ``values`` over the tokens where ``mask`` is set.

    ``out = (x - mean) / (std + eps)`` with the mean and population standard
    deviation taken over masked tokens, and 0 at unmasked positions.  The
    reference has no such function; this is the definition this package uses
    for whitened PPO advantages (``shift_mean=False`` only rescales).
    """

    if values.shape != mask.shape:
        raise ValueError("values and mask must have the same shape")
    if not values.is_floating_point():
        raise TypeError("values must be floating point")
    if eps < 0:
        raise ValueError("eps must be non-negative")
    dev = nat.require_device(values)
    m = mask if mask.device == dev else mask.to(dev)
    B, T = nat.flatten_rows(values.shape)
    xv, _xk = nat.rows_view(values, B, T)
    mv, _mk = nat.rows_view(m, B, T)
    acc = nat.acc_dtype(values.dtype)
    ws = torch.empty(nat.lib().rrl_reduce_workspace_bytes(B * T), dtype=torch.uint8, device=dev)
    out = torch.empty(values.shape, dtype=acc, device=dev)
    status = nat.new_status(dev)
    nat.call("rrl_masked_whiten", B, T, xv, mv, float(eps), int(bool(shift_mean)),
             nat.dtype_code(acc), ws.data_ptr(), out.data_ptr(), nat.dtype_code(acc),
             status.data_ptr(), nat.stream_ptr(dev))
    if nat.read_status(status) & nat.FLAG_EMPTY_MASK:
        raise ValueError("cannot reduce an empty mask")
    return out.to(values.dtype)
