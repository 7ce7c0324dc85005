"""ctypes binding of ``librosellm_amd.so`` (declared in ``include/roserlhf_amd.h``).

This module is the only bridge between the Python API and the gfx950 kernels.
It fails loudly: a missing library raises ``ImportError`` at import time of
the API modules' first call, and there is no CPU fallback anywhere in the
package.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional, Sequence, Tuple

import torch

LIB_PATH = Path(__file__).resolve().parent / "librosellm_amd.so"

# rrl_dtype codes
F32, F64, BF16, F16, BOOL, U8, I8, I16, I32, I64 = range(10)

_TORCH_TO_CODE = {
    torch.float32: F32,
    torch.float64: F64,
    torch.bfloat16: BF16,
    torch.float16: F16,
    torch.bool: BOOL,
    torch.uint8: U8,
    torch.int8: I8,
    torch.int16: I16,
    torch.int32: I32,
    torch.int64: I64,
}

# rrl_flag bits
FLAG_EMPTY_MASK = 1
FLAG_EMPTY_ROW = 2
FLAG_TARGET_RANGE = 4
FLAG_INVALID_TURN = 8
FLAG_FAST_RANGE = 16
FLAG_BAD_PROBS = 32
FLAG_LM_RANGE = 64

# rrl_policy_flag
POLICY_GENERIC = 1
POLICY_SKIP_MASKED = 2
POLICY_SUM = 4
POLICY_RERUN_FAST_RANGE = 8

# rrl_objective
OBJ_PPO, OBJ_SAO, OBJ_GSPO, OBJ_GSPO_TOKEN, OBJ_SAPO, OBJ_NLL = range(6)
NSCALARS = 8


class RrlView(ctypes.Structure):
    _fields_ = [
        ("ptr", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("s_row", ctypes.c_int64),
        ("s_col", ctypes.c_int64),
    ]


class RrlPolicyParams(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("detach_ratio", ctypes.c_int32),
        ("mask_is_weight", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("clip_low", ctypes.c_double),
        ("clip_high", ctypes.c_double),
        ("max_log_ratio", ctypes.c_double),
        ("tau_positive", ctypes.c_double),
        ("tau_negative", ctypes.c_double),
        ("ignore_index", ctypes.c_int64),
    ]


_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_D = ctypes.c_double
_V = RrlView
_PP = ctypes.POINTER(RrlPolicyParams)

# name -> (restype, argtypes); mirrors include/roserlhf_amd.h
SIGNATURES = {
    "rrl_last_error": (ctypes.c_char_p, []),
    "rrl_abi_version": (ctypes.c_int, []),
    "rrl_logprob_fwd": (ctypes.c_int, [_P, _I32, _I64, _I64, _I64, _I64, _I64, _V, _P, _I32, _P, _P, _P]),
    "rrl_logprob_fwd_masked": (ctypes.c_int, [_P, _I32, _I64, _I64, _I64, _I64, _I64, _V, _V, _P, _I32, _P, _P, _P]),
    "rrl_logprob_bwd": (ctypes.c_int, [_P, _I32, _I64, _I64, _I64, _I64, _I64, _V, _P, _P, _P, _P, _I32, _I64, _I64, _I32, _P]),
    "rrl_scale_rows": (ctypes.c_int, [_P, _I32, _I64, _I64, _I64, _I64, _I64, _P, _I32, _D, _P]),
    "rrl_policy_workspace_bytes": (ctypes.c_size_t, [_I64, _I32]),
    "rrl_policy_fwd": (ctypes.c_int, [_PP, _I64, _I64, _V, _V, _V, _V, _I32, _P, _P, _P, _P, _P, _P]),
    "rrl_policy_bwd": (ctypes.c_int, [_PP, _I64, _I64, _V, _V, _V, _V, _I32, _P, _P, _P, _P, _P]),
    "rrl_policy_row_coef": (ctypes.c_int, [_PP, _I64, _I64, _V, _I32, _P, _P, _P, _P]),
    "rrl_fused_records_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "rrl_check_targets": (ctypes.c_int, [_PP, _I64, _I64, _I64, _V, _P, _P]),
    "rrl_fused_logprob_policy": (ctypes.c_int, [_PP, _P, _I32, _I64, _I64, _I64, _I64, _I64, _V, _V, _V, _V, _P, _P, _P, _P, _P, _I32, _I64, _I64, _P, _P]),
    "rrl_fused_logprob_policy_noalloc": (ctypes.c_int, [_PP, _P, _I32, _I64, _I64, _I64, _I64, _I64, _V, _V, _V, _V, _P, _P, _P, _P, _I32, _I64, _I64, _P, _P]),
    "rrl_reduce_workspace_bytes": (ctypes.c_size_t, [_I64]),
    "rrl_masked_mean_fwd": (ctypes.c_int, [_I64, _I64, _V, _V, _I32, _P, _P, _P, _P]),
    "rrl_masked_mean_bwd": (ctypes.c_int, [_I64, _I64, _V, _I32, _P, _P, _P, _P]),
    "rrl_sequence_log_ratio_fwd": (ctypes.c_int, [_I64, _I64, _V, _V, _V, _I32, _I32, _P, _P, _P, _P]),
    "rrl_sequence_log_ratio_bwd": (ctypes.c_int, [_I64, _I64, _V, _I32, _I32, _P, _P, _P, _P]),
    "rrl_double_sided_mask": (ctypes.c_int, [_I64, _P, _I32, _D, _D, _P, _P]),
    "rrl_discounted_returns": (ctypes.c_int, [_I64, _I64, _V, _V, _V, _V, _D, _P, _I32, _P]),
    "rrl_gae": (ctypes.c_int, [_I64, _I64, _V, _V, _V, _V, _V, _D, _D, _P, _P, _I32, _P]),
    "rrl_skip_observation_gae": (ctypes.c_int, [_I64, _I64, _V, _V, _V, _V, _V, _D, _D, _P, _P, _I32, _P]),
    "rrl_group_standardize": (ctypes.c_int, [_I64, _I64, _V, _D, _P, _I32, _P]),
    "rrl_leave_one_out": (ctypes.c_int, [_I64, _I64, _V, _P, _I32, _P]),
    "rrl_broadcast_turn": (ctypes.c_int, [_I64, _I64, _I64, _V, _V, _V, _P, _I32, _P, _P]),
    "rrl_masked_whiten": (ctypes.c_int, [_I64, _I64, _V, _V, _D, _I32, _I32, _P, _P, _I32, _P, _P]),
    "rrl_sample_logprobs": (ctypes.c_int, [_P, _I32, _I64, _I64, _I64, _D, _I64, _D, _I32,
                                           ctypes.c_uint64, ctypes.c_uint64, _P, _P, _P, _P, _P]),
    "rrl_lm_head_fwd_workspace_bytes": (ctypes.c_size_t, [_I64]),
    "rrl_lm_head_fwd": (ctypes.c_int, [_P, _P, _I32, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _I64, _P, _P, _P]),
    "rrl_lm_head_dhidden": (ctypes.c_int, [_P, _I32, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _P, _I64, _P]),
    "rrl_lm_head_dweight_workspace_bytes": (ctypes.c_size_t, [_I64, _I64, _I64]),
    "rrl_lm_head_dweight": (ctypes.c_int, [_P, _P, _I32, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _I32, _I64, _P]),
    "rrl_transpose16": (ctypes.c_int, [_P, _I64, _I64, _I64, _P, _I64, _P]),
    "rrl_philox4x32_10": (None, [ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32)]),
}

_lib: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise ImportError when it is absent."""

    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"rosellm_amd: {LIB_PATH.name} is not built; run `python -m rosellm_amd.build` "
            "(hipcc, gfx950). There is no CPU fallback."
        )
    lib = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_GLOBAL)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


def lib() -> ctypes.CDLL:
    return _lib if _lib is not None else load()


# Optional per-entry-point launch timing: name -> list of (start, end)
# torch.cuda.Event pairs recorded on the stream the call is launched on.
_timed: dict = {}
_event_pool: list = []


def time_calls(*names: str, capacity: int = 0) -> dict:
    """Record a HIP event pair around every later call of each named entry
    point (on torch's current stream, where the call launches its kernels).
    ``capacity`` calls' events are created up front, so that recording adds
    only the two event records to a timed call.  Returns the live
    name -> [(start, end), ...] mapping; ``time_calls()`` with no names stops
    recording."""

    global _timed, _event_pool
    _timed = {n: [] for n in names}
    _event_pool = [torch.cuda.Event(enable_timing=True) for _ in range(2 * capacity)]
    return _timed


def _event() -> "torch.cuda.Event":
    return _event_pool.pop() if _event_pool else torch.cuda.Event(enable_timing=True)


class _TimedSpan:
    """HIP event pair around a block of torch work (a library GEMM) when
    ``name`` is being recorded by ``time_calls``."""

    __slots__ = ("events", "start")

    def __init__(self, name: str):
        self.events = _timed.get(name) if _timed else None
        self.start = None

    def __enter__(self):
        if self.events is not None:
            self.start = _event()
            self.start.record()
        return self

    def __exit__(self, *exc):
        if self.events is not None:
            end = _event()
            end.record()
            self.events.append((self.start, end))
        return False


def timed(name: str) -> _TimedSpan:
    """Context manager: ``with timed("lm_logits_gemm"): torch.mm(...)`` records
    the span under that name while ``time_calls`` records it."""

    return _TimedSpan(name)


def call(name: str, *args, timed: bool = True) -> None:
    """Call an entry point and raise on a non-zero return code.  ``timed=False``
    keeps the call out of ``time_calls``' records: a launch that is not the
    entry point's own work (the conditional rerun behind a single-pass sweep)."""

    events = _timed.get(name) if _timed and timed else None
    if events is not None:
        start = _event()
        start.record()
    rc = getattr(lib(), name)(*args)
    if events is not None:
        end = _event()
        end.record()
        events.append((start, end))
    if rc != 0:
        msg = lib().rrl_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


# ---------------------------------------------------------------------------
# Tensor plumbing
# ---------------------------------------------------------------------------


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _TORCH_TO_CODE[dtype]
    except KeyError:
        raise TypeError(f"rosellm_amd: unsupported dtype {dtype}") from None


def require_device(*tensors: Optional[torch.Tensor]) -> torch.device:
    """All tensors must live on one ROCm device; the kernels have no CPU path."""

    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "rosellm_amd.roserlhf runs its kernels on a ROCm GPU; got a tensor on "
                f"'{t.device}'. Move inputs to the GPU (there is no CPU fallback)."
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors are on different devices: {dev} and {t.device}")
    if dev is None:
        raise RuntimeError("rosellm_amd: no tensor argument to infer the device from")
    return dev


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device: torch.device) -> int:
    """The current HIP stream of `device` as an integer handle.  torch's raw
    accessor skips building a Stream object (about 2 us per call, paid by
    every entry point); the public call is the fallback."""

    if _raw_stream is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(idx)
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


NONE_VIEW = RrlView(None, F32, 0, 0)


def rows_view(t: torch.Tensor, B: int, T: int) -> Tuple[RrlView, torch.Tensor]:
    """A [B, T] strided view of ``t`` (whose elements number B*T).

    Keeps expand()/slice views without copying when their layout is expressible
    with two strides; otherwise falls back to a contiguous copy.  Returns the
    view and the tensor that must stay alive for the duration of the call.
    """

    if t.dim() == 2 and tuple(t.shape) == (B, T):
        return RrlView(t.data_ptr(), dtype_code(t.dtype), t.stride(0), t.stride(1)), t
    if t.dim() == 1 and B == 1 and t.shape[0] == T:
        return RrlView(t.data_ptr(), dtype_code(t.dtype), 0, t.stride(0)), t
    if t.dim() == 0 and B * T == 1:
        return RrlView(t.data_ptr(), dtype_code(t.dtype), 0, 0), t
    try:
        v = t.view(B, T)
    except RuntimeError:
        v = t.reshape(B, T)
    return RrlView(v.data_ptr(), dtype_code(v.dtype), v.stride(0), v.stride(1)), v


def vector_view(t: torch.Tensor) -> Tuple[RrlView, torch.Tensor]:
    """A length-B operand broadcast over columns (s_col = 0)."""

    v = t.reshape(-1)
    return RrlView(v.data_ptr(), dtype_code(v.dtype), v.stride(0), 0), v


def flatten_rows(shape: Sequence[int]) -> Tuple[int, int]:
    """(B, T) for a [..., T] shape: leading dims collapse into B."""

    if len(shape) == 0:
        return 1, 1
    T = int(shape[-1])
    B = 1
    for s in shape[:-1]:
        B *= int(s)
    return B, T


def logits_rows(logits: torch.Tensor) -> Tuple[torch.Tensor, int, int, int, int, int]:
    """Describe logits [..., V] as rows (b, t) with two row strides.

    Returns (tensor, B, T, V, stride_b, stride_t).  The vocabulary must be
    contiguous; prefix dims beyond two are merged when their strides allow it.
    """

    x = logits if logits.stride(-1) == 1 else logits.contiguous()
    V = x.shape[-1]
    prefix = list(x.shape[:-1])
    if len(prefix) == 1:
        return x, 1, prefix[0], V, 0, x.stride(0)
    B, T = flatten_rows(prefix)
    # reshape() returns a view whenever the leading dims merge with one stride.
    y = x.reshape(B, T, V)
    if y.stride(-1) != 1:
        y = y.contiguous()
    return y, B, T, V, y.stride(0), y.stride(1)


def acc_dtype(*dtypes: torch.dtype) -> torch.dtype:
    return torch.float64 if any(d == torch.float64 for d in dtypes) else torch.float32


def new_status(device: torch.device) -> torch.Tensor:
    return torch.zeros(1, dtype=torch.int32, device=device)


def read_status(status: torch.Tensor) -> int:
    return int(status.item())
