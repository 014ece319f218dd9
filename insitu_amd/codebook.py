"""Codebook: the integers the device compares against and multiplies by.

Mirrors ops/codebook.py:33-180 of the reference. The Lloyd-Max solve is a
one-off host computation (it runs once per width per process); the device
receives the resulting integers through the cache descriptor, as the RTL
receives them as parameters (hw/vectors.py:427-431).
"""

from __future__ import annotations

import functools
from dataclasses import dataclass

import numpy as np


def _q_from_float(x, frac: int, width: int = 32) -> np.ndarray:
    """Q(width, frac).from_float: rint (half-even) then saturate (numerics/fixed.py:137-164)."""
    r = np.rint(np.asarray(x, dtype=np.float64) * (1 << frac)).astype(np.int64)
    return np.clip(r, -(1 << (width - 1)), (1 << (width - 1)) - 1)


def _strictly_ascending(a: np.ndarray) -> np.ndarray:
    """codebook.py:165-180."""
    a = a.astype(np.int64).copy()
    for i in range(1, len(a)):
        if a[i] <= a[i - 1]:
            a[i] = a[i - 1] + 1
    return a


@dataclass(frozen=True)
class Codebook:
    centroids: np.ndarray      # (2**bits,) int64, Q(frac), ascending
    boundaries: np.ndarray     # (2**bits - 1,) int64
    bits: int
    frac: int

    def __post_init__(self) -> None:
        n = 1 << self.bits
        if self.centroids.shape != (n,) or self.boundaries.shape != (n - 1,):
            raise ValueError("codebook shape does not match its width")
        if not (np.all(np.diff(self.centroids) > 0) and np.all(np.diff(self.boundaries) > 0)):
            raise ValueError("centroids and boundaries must be strictly ascending")

    @property
    def size(self) -> int:
        return 1 << self.bits

    def to_float(self) -> np.ndarray:
        return self.centroids.astype(np.float64) / (1 << self.frac)

    @staticmethod
    @functools.lru_cache(maxsize=64)
    def gaussian(bits: int, frac: int = 15, symmetric: bool = True,
                 grid: int = 1 << 16, iters: int = 200) -> "Codebook":
        """Lloyd-Max for N(0,1) on a 65,536-point grid over [-8, 8] (codebook.py:67-120)."""
        if bits < 1:
            raise ValueError(f"bits={bits} must be at least 1")
        n = 1 << bits
        x = np.linspace(-8.0, 8.0, grid)
        w = np.exp(-0.5 * x * x)
        w /= w.sum()
        cdf = np.cumsum(w)
        c = np.interp((np.arange(n) + 0.5) / n, cdf, x)      # equiprobable start
        for _ in range(iters):
            mid = 0.5 * (c[:-1] + c[1:])
            cell = np.searchsorted(mid, x)
            mass = np.bincount(cell, weights=w, minlength=n)
            first = np.bincount(cell, weights=w * x, minlength=n)
            nxt = np.where(mass > 0, first / np.maximum(mass, 1e-300), c)
            done = np.allclose(nxt, c, atol=1e-12)
            c = nxt
            if done:
                break
        if symmetric:
            c = 0.5 * (c - c[::-1])
        cq = _strictly_ascending(_q_from_float(c, frac))
        # Midpoints floored: a value exactly on a boundary goes to the lower bin.
        bq = _strictly_ascending((cq[:-1] + cq[1:]) >> np.int64(1))
        return Codebook(centroids=cq, boundaries=bq, bits=bits, frac=frac)

    @staticmethod
    @functools.lru_cache(maxsize=64)
    def uniform(bits: int, frac: int = 15, symmetric: bool = True,
                grid: int = 1 << 16) -> "Codebook":
        """MSE-optimal equally spaced levels, clipping range scanned (codebook.py:123-154)."""
        n = 1 << bits
        x = np.linspace(-8.0, 8.0, grid)
        w = np.exp(-0.5 * x * x)
        w /= w.sum()
        best, best_mse = None, np.inf
        for c in np.linspace(0.5, 6.0, 400):
            levels = np.linspace(-c, c, n) if n > 1 else np.array([0.0])
            edges = 0.5 * (levels[:-1] + levels[1:])
            mse = float((w * (levels[np.searchsorted(edges, x)] - x) ** 2).sum())
            if mse < best_mse:
                best, best_mse = levels, mse
        cq = _strictly_ascending(_q_from_float(best, frac))
        bq = _strictly_ascending((cq[:-1] + cq[1:]) >> np.int64(1))
        return Codebook(centroids=cq, boundaries=bq, bits=bits, frac=frac)

    @staticmethod
    def build(kind: str, bits: int, frac: int = 15, symmetric: bool = True) -> "Codebook":
        if kind == "gaussian":
            return Codebook.gaussian(bits, frac, symmetric)
        if kind == "uniform":
            return Codebook.uniform(bits, frac, symmetric)
        raise ValueError(f"unknown codebook {kind!r}")
