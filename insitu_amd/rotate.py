"""Rotation: the randomized Hadamard transform, applied on the GPU.

Mirrors ops/rotate.py:107-197 of the reference. The sign diagonal is drawn
from PCG64(seed) exactly as rotate.py:153-154 draws it (numpy's own
generator), and is handed to the device as one bit word per round, bit i set
meaning channel i is negated (the format of tb/vectors/rot_signs.hex).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from .runtime import default_context, ptr


def sqrt_shift(n: int):
    """numerics/fixed.py:229-240."""
    if n < 1 or n & (n - 1):
        return None
    e = n.bit_length() - 1
    return e // 2 if e % 2 == 0 else None


@dataclass(frozen=True)
class Rotation:
    d: int
    signs: np.ndarray     # (rounds, d) int64 +-1
    seed: int

    @property
    def rounds(self) -> int:
        return self.signs.shape[0]

    @staticmethod
    def for_quant(quant, d: int) -> "Rotation":
        return Rotation.from_seed(d, quant.seed, quant.rot_rounds)

    @staticmethod
    def from_seed(d: int, seed: int, rounds: int = 1) -> "Rotation":
        if d & (d - 1):
            raise ValueError(f"d={d} must be a power of two for a Hadamard butterfly")
        if rounds < 0:
            raise ValueError(f"rounds={rounds} must not be negative")
        rng = np.random.Generator(np.random.PCG64(seed))
        signs = rng.integers(0, 2, size=(rounds, d)).astype(np.int64) * 2 - 1
        return Rotation(d=d, signs=signs, seed=seed)

    @property
    def shift(self):
        return sqrt_shift(self.d)

    def sign_words(self) -> list[tuple[int, int]]:
        """Per round (channels 0..63, channels 64..127) bit words; bit set = negate."""
        out = []
        for row in self.signs:
            w = [0, 0]
            for i, s in enumerate(row):
                if s < 0:
                    w[i // 64] |= 1 << (i % 64)
            out.append((w[0], w[1]))
        return out

    def matrix(self) -> np.ndarray:
        """rotate.py:233-251: the dense float64 form R_last ... R_0 (H * signs / sqrt d
        per round, round 0 applied first), for folding into W_o; never on a hot path."""
        h = np.array([[1.0]])
        while h.shape[0] < self.d:
            h = np.block([[h, h], [h, -h]])
        m = np.eye(self.d)
        for r in range(self.rounds):
            m = ((h * self.signs[r]) / np.sqrt(self.d)) @ m
        return m

    def fill_format(self, f: "_lib.Format") -> None:
        if self.rounds > 8:
            raise ValueError("at most 8 rotation rounds fit the descriptor")
        f.rot_rounds = self.rounds
        for r, (a, b) in enumerate(self.sign_words()):
            f.rot_signs[r][0] = a
            f.rot_signs[r][1] = b

    def apply(self, x, ctx=None):
        """Rotate along the last axis on the device. Returns a torch int32 tensor.

        rotate.py:170-197: per round fwht(x * signs) then the 1/sqrt(d) scale
        (floor). Input must be within int32 (the seam carries 24 bits).
        """
        import torch
        ctx = ctx or default_context()
        a = ctx.to_device(x, torch.int32)
        if a.shape[-1] != self.d:
            raise ValueError(f"rotate expects last axis {self.d}, got {a.shape[-1]}")
        out = torch.empty_like(a)
        f = _lib.Format()
        f.head_dim = self.d
        self.fill_format(f)
        n = a.numel() // self.d
        _lib.check(ctx.lib.insitu_rotate(ctx.handle, ptr(a), ptr(out), n, ctypes.byref(f)))
        return out
