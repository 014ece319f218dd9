"""Synthetic seam inputs for the benchmark configurations.

The reference has no generator for this distribution, so it is defined here
(and stated in the design notes):

    rng = numpy.random.default_rng(seed)
    outliers: per head, chosen once, in the order q heads, k heads, v heads:
        C0-C3: rng.choice(d, 4, replace=False), scaled x8
        C4:    each channel independently with p = 0.01, scaled x16
    steps: q (n, Hq, d), k (n, Hkv, d), v (n, Hkv, d) drawn in that order as
        float32 rng.standard_normal, then the outlier channels scaled
    to_fixed: rint(x * 2^16) (half-even), saturate to 24 bits (ops/convert.py:44-57)

q carries no 1/sqrt(d) pre-scale (the configurations say ~N(0,1) post-RoPE).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

QK_FRAC = 16
QK_WIDTH = 24


def to_fixed(x, frac: int = QK_FRAC, width: int = QK_WIDTH) -> np.ndarray:
    """ops/convert.py:44-57: fp -> Q(frac) ints, half-even, saturating."""
    r = np.rint(np.asarray(x, dtype=np.float64) * (1 << frac)).astype(np.int64)
    return np.clip(r, -(1 << (width - 1)), (1 << (width - 1)) - 1)


@dataclass
class Workload:
    n_q_heads: int = 32
    n_kv_heads: int = 8
    head_dim: int = 64
    seed: int = 0
    outlier_mode: str = "four"      # "four" (C0-C3) or "percent" (C4)
    batch: int = 1

    def __post_init__(self) -> None:
        self.rng = np.random.default_rng(self.seed)
        d = self.head_dim
        scale = np.ones((self.n_q_heads + 2 * self.n_kv_heads, d), dtype=np.float32)
        for h in range(scale.shape[0]):
            if self.outlier_mode == "four":
                scale[h, self.rng.choice(d, 4, replace=False)] = 8.0
            elif self.outlier_mode == "percent":
                scale[h, self.rng.random(d) < 0.01] = 16.0
            else:
                raise ValueError(self.outlier_mode)
        self.q_scale = scale[:self.n_q_heads]
        self.k_scale = scale[self.n_q_heads:self.n_q_heads + self.n_kv_heads]
        self.v_scale = scale[self.n_q_heads + self.n_kv_heads:]

    def steps(self, n: int):
        """n tokens of wire q/k/v for every sequence: int64 arrays
        q (batch, n, Hq, d), k (batch, n, Hkv, d), v (batch, n, Hkv, d)."""
        b, d = self.batch, self.head_dim
        q = self.rng.standard_normal((b, n, self.n_q_heads, d), dtype=np.float32) * self.q_scale
        k = self.rng.standard_normal((b, n, self.n_kv_heads, d), dtype=np.float32) * self.k_scale
        v = self.rng.standard_normal((b, n, self.n_kv_heads, d), dtype=np.float32) * self.v_scale
        return to_fixed(q), to_fixed(k), to_fixed(v)
