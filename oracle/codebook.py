"""Lloyd-Max scalar codebooks for N(0,1), stored Q(frac) (oracle; test infrastructure only).

Restates ops/codebook.py:67-180 of the reference. The float solve follows the
same numpy calls in the same order, so on the same numpy build it lands on
the same integers; the 2- and 4-bit results are pinned by tb/vectors.
"""

from __future__ import annotations

import functools

import numpy as np

from .fixed import I64, Q


def _strictly_ascending(a: np.ndarray) -> np.ndarray:
    """ops/codebook.py:165-180: nudge ties introduced by rounding upward by one."""
    a = a.astype(I64).copy()
    for i in range(1, len(a)):
        if a[i] <= a[i - 1]:
            a[i] = a[i - 1] + 1
    return a


@functools.lru_cache(maxsize=64)
def gaussian(bits: int, frac: int = 15, symmetric: bool = True,
             grid: int = 1 << 16, iters: int = 200):
    """ops/codebook.py:67-120. Returns (centroids, boundaries) as int64 arrays."""
    if bits < 1:
        raise ValueError("bits must be at least 1")
    n = 1 << bits
    x = np.linspace(-8.0, 8.0, grid)
    w = np.exp(-0.5 * x * x)
    w /= w.sum()
    cdf = np.cumsum(w)
    c = np.interp((np.arange(n) + 0.5) / n, cdf, x)
    for _ in range(iters):
        b = 0.5 * (c[:-1] + c[1:])
        region = np.searchsorted(b, x)
        mass = np.bincount(region, weights=w, minlength=n)
        moment = np.bincount(region, weights=w * x, minlength=n)
        new = np.where(mass > 0, moment / np.maximum(mass, 1e-300), c)
        if np.allclose(new, c, atol=1e-12):
            c = new
            break
        c = new
    if symmetric:
        c = 0.5 * (c - c[::-1])
    cq = _strictly_ascending(Q(32, frac).from_float(c))
    bq = _strictly_ascending((cq[:-1] + cq[1:]) >> I64(1))
    return cq, bq
