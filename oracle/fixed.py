"""Fixed-point primitives (oracle; test infrastructure only).

Restates numerics/fixed.py of the reference: the three right-shift rounding
rules, saturating Q formats, the unnormalised integer Walsh-Hadamard transform
and the exact-shift test for 1/sqrt(d).
"""

from __future__ import annotations

import math

import numpy as np

I64 = np.int64


def as_int(x) -> np.ndarray:
    a = np.asarray(x)
    if a.dtype.kind not in "iu":
        raise TypeError(f"fixed-point op on dtype {a.dtype}")
    return a.astype(I64, copy=False)


def rshift(x, n, rounding: str = "floor") -> np.ndarray:
    """x >> n under `rounding` in {"floor", "even", "up"}; numerics/fixed.py:49-89.

    floor is the arithmetic shift; "up" adds half then floors; "even" adds half,
    floors, and clears bit 0 when the discarded bits were exactly one half.
    `n` may be an array (per-row shifts, as the reciprocal needs).
    """
    a = as_int(x)
    scalar = np.ndim(n) == 0
    if scalar:
        n = int(n)
        if n < 0:
            raise ValueError("negative right shift")
        if n == 0:
            return a
        nn = I64(n)
        half = I64(1) << I64(n - 1)
    else:
        nn = as_int(n)
        if np.any(nn < 0):
            raise ValueError("negative right shift")
        half = I64(1) << (np.maximum(nn, 1) - 1)
    if rounding == "floor":
        return a >> nn
    if rounding not in ("up", "even"):
        raise ValueError(f"unknown rounding {rounding!r}")
    q = (a + half) >> nn
    if rounding == "even":
        tie = (a & ((I64(1) << nn) - 1)) == half
        q = np.where(tie, q & ~I64(1), q)
    if not scalar:
        q = np.where(nn == 0, a, q)
    return q


def lshift(x, n: int) -> np.ndarray:
    return as_int(x) << I64(n)


class Q:
    """Signed two's-complement format; numerics/fixed.py:111-199."""

    def __init__(self, width: int, frac: int, saturate: bool = True) -> None:
        if width < 2 or not 0 <= frac < width:
            raise ValueError("bad Q format")
        self.width, self.frac, self.saturate = width, frac, saturate

    @property
    def lo(self) -> int:
        return -(1 << (self.width - 1))

    @property
    def hi(self) -> int:
        return (1 << (self.width - 1)) - 1

    def clamp(self, x) -> np.ndarray:
        a = as_int(x)
        if not self.saturate:
            span = I64(1) << I64(self.width)
            off = I64(1) << I64(self.width - 1)
            return ((a + off) % span) - off
        return np.clip(a, self.lo, self.hi)

    def overflow_count(self, x) -> int:
        a = as_int(x)
        return int(((a < self.lo) | (a > self.hi)).sum())

    def from_float(self, x, rounding: str = "even") -> np.ndarray:
        """fixed.py:137-153: scale by 2^frac, round (rint is half-even), clamp."""
        a = np.asarray(x, dtype=np.float64) * (1 << self.frac)
        if rounding == "even":
            r = np.rint(a)
        elif rounding == "up":
            r = np.floor(a + 0.5)
        elif rounding == "floor":
            r = np.floor(a)
        else:
            raise ValueError(rounding)
        return self.clamp(r.astype(I64))

    def requantize(self, x, src_frac: int, rounding: str = "floor") -> np.ndarray:
        """fixed.py:189-196: move from Q(src_frac) to this format, then clamp."""
        s = src_frac - self.frac
        if s > 0:
            x = rshift(x, s, rounding)
        elif s < 0:
            x = lshift(x, -s)
        return self.clamp(x)


def fwht(x) -> np.ndarray:
    """Unnormalised WHT on the last axis, stages h = 1, 2, 4, ...; fixed.py:202-226.

    Stage h pairs element i (bit h clear) with i + h: new[i] = a + b,
    new[i + h] = a - b.
    """
    a = as_int(x).copy()
    n = a.shape[-1]
    if n & (n - 1):
        raise ValueError(f"fwht length {n} is not a power of two")
    h = 1
    while h < n:
        v = a.reshape(*a.shape[:-1], n // (2 * h), 2, h)
        lo = v[..., 0, :].copy()
        hi = v[..., 1, :].copy()
        v[..., 0, :] = lo + hi
        v[..., 1, :] = lo - hi
        a = v.reshape(*a.shape[:-1], n)
        h *= 2
    return a


def sqrt_shift(n: int):
    """log2(sqrt(n)) when it is a whole number, else None; fixed.py:229-240."""
    if n < 1 or n & (n - 1):
        return None
    e = n.bit_length() - 1
    return e // 2 if e % 2 == 0 else None


def inv_sqrt_q15(n: int) -> int:
    """round(2^15 / sqrt(n)); fixed.py:243-246 (Python round, half-even)."""
    return int(round((1 << 15) / math.sqrt(n)))
