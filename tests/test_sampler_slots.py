"""The register-resident nucleus path's slot arithmetic, on the CPU, for every
16-bit pattern.

The top-p counts of ``sample_blocks_kernel`` (rosellm_amd/csrc/sampler.hip,
``slot4``) index a key's count by its ordered key minus the lowest counted
key, klo.  The kernel forms 4 x that slot from the raw bfloat16 bits in one
multiply-add: ``v_mad_u32_u16(bits, 4, 4 (0x8000 - klo))`` when every counted
key is a positive number's (klo > 0x8000), ``v_mad_i32_i16(bits, -4,
4 (-1 - klo))`` (the bits as a signed 16-bit value) when every one is a
negative number's (kmax < 0x8000), and a lane past the row's end takes the
constant 0xfff00000 or 0x80000000.  Here the two instructions' arithmetic
(32-bit wrap-around) is checked against the order-preserving key itself
(``float_key``: +-0 share +0's key, negative values below positive), which
is how the streaming kernel and the tests' key spans rank values:

* an entry is counted (slot below 4 R, R = kmax - klo + 1) exactly when its
  key lies in [klo, kmax], and then its slot is 4 (key - klo);
* a lane past the row's end is never counted and reads past slot R + 1;
* the key order matches the float order of the values (numpy's bfloat16
  widening), so the counts ordered by key are the values in descending
  order.
"""

from __future__ import annotations

import numpy as np
import pytest

BITS = np.arange(1 << 16, dtype=np.int64)
M32 = (1 << 32) - 1


def float_key(b):
    """The kernels' order-preserving 16-bit key (float_key<16>)."""

    b = np.where((b & 0x7FFF) == 0, 0, b)
    return np.where(b & 0x8000, (~b) & 0xFFFF, b | 0x8000)


def mad_u32_u16(b, mul, c):
    return ((b & 0xFFFF) * mul + c) & M32


def mad_i32_i16(b, mul, c):
    s = np.where(b & 0x8000, (b & 0xFFFF) - (1 << 16), b & 0xFFFF)
    return (s * mul + c) & M32


def slots(b, klo, pos, in_row=True):
    if pos:
        c = (4 * (0x8000 - klo)) & M32 if in_row else 0xFFF00000
        return mad_u32_u16(b, 4, c)
    c = (4 * (0xFFFFFFFF - klo)) & M32 if in_row else 0x80000000
    return mad_i32_i16(b, -4, c)


def _cases():
    # (klo, kmax) pairs the kernel takes: positive ranges (klo > 0x8000)
    # and negative ones (kmax < 0x8000), narrow and up to 4096 keys wide,
    # at both ends of each half.
    out = []
    for klo, kmax in [(0x8001, 0x8001), (0x8001, 0x8FFF), (0xBF80, 0xC100), (0xC0A0, 0xC29F),
                      (0xF000, 0xFF7F), (0xFF7F, 0xFF7F), (0xEF80, 0xFF7F)]:
        out.append((klo, kmax, True))
    for klo, kmax in [(0x0001, 0x0FFF), (0x007F, 0x107E), (0x3E00, 0x3F7F), (0x7000, 0x7FFE),
                      (0x7FFE, 0x7FFE), (0x0080, 0x0080)]:
        out.append((klo, kmax, False))
    return out


@pytest.mark.parametrize("klo,kmax,pos", _cases())
def test_slot_is_key_minus_klo(klo, kmax, pos):
    assert kmax - klo < 4096
    assert (klo > 0x8000) if pos else (kmax < 0x8000)
    R = kmax - klo + 1
    key = float_key(BITS)
    t = slots(BITS, klo, pos)
    counted = t < 4 * R
    inside = (key >= klo) & (key <= kmax)
    bad = np.nonzero(counted != inside)[0]
    assert bad.size == 0, f"bits {bad[:8]} counted {counted[bad[:8]]} keys {key[bad[:8]]}"
    assert np.array_equal(t[inside], 4 * (key[inside] - klo))
    # The fixed slots R (entries below klo, weight 1e-9) and R + 1 (lanes
    # past the row's end, weight 0) are reached only through the clamp.
    assert (t[~inside] >= 4 * R).all()


@pytest.mark.parametrize("klo,kmax,pos", _cases())
def test_lanes_past_the_row_are_never_counted(klo, kmax, pos):
    R = kmax - klo + 1
    t = slots(BITS, klo, pos, in_row=False)
    assert (t >= 4 * (R + 2)).all()


def test_key_order_is_value_order():
    """Ascending key = ascending value over every non-NaN bfloat16 pattern
    (+-0 equal), so 'the counts in descending key order' are the row's
    values in descending order."""

    vals = (BITS.astype(np.uint32) << 16).view(np.float32)
    ok = ~np.isnan(vals)
    keys = float_key(BITS)[ok]
    v = vals[ok]
    order = np.argsort(keys, kind="stable")
    assert np.all(np.diff(v[order]) >= 0)
    # equal keys exactly when the values are equal (only +-0 share one)
    same = np.diff(keys[order]) == 0
    assert np.array_equal(same, np.diff(v[order]) == 0)
    assert same.sum() == 1
