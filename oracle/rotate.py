"""Randomized Hadamard rotation R = H.D / sqrt(d) (oracle; test infrastructure only).

Restates ops/rotate.py:124-197 of the reference.
"""

from __future__ import annotations

import numpy as np

from .fixed import I64, fwht, inv_sqrt_q15, rshift, sqrt_shift


def signs_from_seed(d: int, seed: int = 0, rounds: int = 1) -> np.ndarray:
    """(rounds, d) of +-1; ops/rotate.py:144-155 (PCG64, one stream for all rounds)."""
    if d & (d - 1):
        raise ValueError(f"d={d} must be a power of two")
    if rounds < 0:
        raise ValueError("rounds must not be negative")
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.integers(0, 2, size=(rounds, d)).astype(I64) * 2 - 1


def sign_words(signs: np.ndarray) -> list[int]:
    """One integer per round, bit i set when channel i is negated (tb/vectors/rot_signs.hex)."""
    return [sum(int(s < 0) << i for i, s in enumerate(row)) for row in np.atleast_2d(signs)]


def rotate(x, signs: np.ndarray) -> np.ndarray:
    """ops/rotate.py:170-197: per round fwht(x * signs[r]) then the 1/sqrt(d) scale (floor)."""
    a = np.asarray(x, dtype=I64)
    signs = np.atleast_2d(signs)
    d = signs.shape[-1]
    if a.shape[-1] != d:
        raise ValueError(f"rotate expects last axis {d}, got {a.shape[-1]}")
    s = sqrt_shift(d)
    out = a
    for r in range(signs.shape[0]):
        out = fwht(out * signs[r])
        out = rshift(out, s) if s is not None else rshift(out * I64(inv_sqrt_q15(d)), 15)
    return out


def inverse_rotate(y, signs: np.ndarray) -> np.ndarray:
    """ops/rotate.py:199-231: rounds reversed, transform then sign, then scale."""
    a = np.asarray(y, dtype=I64)
    signs = np.atleast_2d(signs)
    d = signs.shape[-1]
    s = sqrt_shift(d)
    out = a
    for r in reversed(range(signs.shape[0])):
        out = fwht(out) * signs[r]
        out = rshift(out, s) if s is not None else rshift(out * I64(inv_sqrt_q15(d)), 15)
    return out


def matrix(signs: np.ndarray) -> np.ndarray:
    """Dense float form, R_last ... R_0 (ops/rotate.py:233-251); for tests."""
    signs = np.atleast_2d(signs)
    d = signs.shape[-1]
    h = np.array([[1.0]])
    while h.shape[0] < d:
        h = np.block([[h, h], [h, -h]])
    m = np.eye(d)
    for r in range(signs.shape[0]):
        m = ((h * signs[r]) / np.sqrt(d)) @ m
    return m
