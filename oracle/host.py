"""The host half of the block either side of the seam, in numpy.

Oracle; test infrastructure only (only tests/, smoke() and bench.py's CPU
baseline read it, as the checker). Restates kernel.py:198-249 and :348-356 of
the reference: the fp16 projections (ops/project.py:21-52, numerics/fp.py:20-62),
the attention scale, RoPE with Llama 3 frequency scaling (ops/rope.py:48-198),
the fp -> fixed cast (ops/convert.py:44-57), the W_o fold (ops/output.py:49-78),
and the seeded synthetic weights (weights.py:112-133) the golden vectors were
made with (hw/vectors.py:821-841).

Pinned by tests/test_oracle_host.py: the projections, the cast and the
fixed-point RoPE reproduce the reference's wire_q/k/v.hex golden rows exactly;
the RoPE scaling regimes and tables by the reference's test_rope_scaling.py
properties; the fold by R^-1 R = I.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .rotate import matrix

QK_FRAC, QK_WIDTH = 16, 24        # config.py:223-224
ROPE_FRAC = 15                    # config.py:225 (centroid_frac): the sin/cos table's format


def to_fp16(x) -> np.ndarray:
    """numerics/fp.py:20-22: round to nearest even."""
    return np.asarray(x, dtype=np.float16)


def project(w, x, bias=None) -> np.ndarray:
    """ops/project.py:21-52 with numerics/fp.py:25-44: x @ w.T in fp16, fp32 products and sums."""
    w16 = to_fp16(w)
    x16 = to_fp16(x)
    out = (w16.astype(np.float32) @ x16.astype(np.float32).T).T.astype(np.float32)
    if bias is not None:
        out = out + np.asarray(bias, dtype=np.float32)
    return out


def to_fixed(x, frac: int = QK_FRAC, width: int = QK_WIDTH):
    """ops/convert.py:44-57: rint (half to even) of x * 2^frac, saturating; (codes, saturated)."""
    r = np.rint(np.asarray(x, dtype=np.float64) * float(1 << frac)).astype(np.int64)
    lo, hi = -(1 << (width - 1)), (1 << (width - 1)) - 1
    sat = int(np.count_nonzero((r < lo) | (r > hi)))
    return np.clip(r, lo, hi), sat


@dataclass(frozen=True)
class RopeScaling:
    """ops/rope.py:48-115: Llama 3's rescaling of inv_freq by wavelength."""

    factor: float
    low_freq_factor: float
    high_freq_factor: float
    original_max_position: int

    def __post_init__(self) -> None:
        if not self.high_freq_factor > self.low_freq_factor:
            raise ValueError("high_freq_factor must exceed low_freq_factor")

    def apply(self, inv_freq) -> np.ndarray:
        f = np.asarray(inv_freq, dtype=np.float64)
        ctx = float(self.original_max_position)
        wavelen = 2.0 * np.pi / f
        low_w, high_w = ctx / self.low_freq_factor, ctx / self.high_freq_factor
        scaled = np.where(wavelen > low_w, f / self.factor, f)
        smooth = (ctx / wavelen - self.low_freq_factor) / (self.high_freq_factor - self.low_freq_factor)
        smoothed = (1.0 - smooth) * scaled / self.factor + smooth * scaled
        between = (wavelen <= low_w) & (wavelen >= high_w)
        return np.where(between, smoothed, scaled)


def rope_tables(d: int, max_position: int, theta: float = 10000.0, frac: int = ROPE_FRAC,
                scaling: RopeScaling | None = None):
    """ops/rope.py:131-142: cos/sin of position * inv_freq in Q(32, frac), half-even."""
    half = d // 2
    inv = 1.0 / (theta ** (np.arange(0, half, dtype=np.float64) * 2.0 / d))
    if scaling is not None:
        inv = scaling.apply(inv)
    ang = np.arange(max_position, dtype=np.float64)[:, None] * inv[None, :]
    q = lambda a: np.clip(np.rint(a * float(1 << frac)), -(1 << 31), (1 << 31) - 1).astype(np.int64)
    return q(np.cos(ang)), q(np.sin(ang))


def rope_fixed(x, positions, cos, sin, frac: int = ROPE_FRAC) -> np.ndarray:
    """ops/rope.py:144-174: half-split pairs, Q(qk + frac) products, one floor shift."""
    a = np.asarray(x, dtype=np.int64)
    half = a.shape[-1] // 2
    c, s = cos[positions], sin[positions]
    lo, hi = a[..., :half], a[..., half:]
    return np.concatenate([(lo * c - hi * s) >> frac, (lo * s + hi * c) >> frac], axis=-1)


def rope_float(x, positions, cos, sin, frac: int = ROPE_FRAC) -> np.ndarray:
    """ops/rope.py:176-198: the same rotation in float64, table over 2^frac."""
    a = np.asarray(x, dtype=np.float64)
    half = a.shape[-1] // 2
    scale = float(1 << frac)
    c, s = cos[positions] / scale, sin[positions] / scale
    lo, hi = a[..., :half], a[..., half:]
    return np.concatenate([lo * c - hi * s, lo * s + hi * c], axis=-1)


def seam(p, n_q: int, n_kv: int, d: int, positions, cos, sin, *, bias=None,
         cast_after_rope: bool = True):
    """kernel.py:209-249 from the fp32 projections p (n, (n_q + 2 n_kv) d) of n tokens:
    split heads, q * 1/sqrt(d) (kernel.py:103, 219), RoPE and the cast in either order.
    Returns wire (q (n, n_q, d), k (n, n_kv, d), v (n, n_kv, d)) int64 and saturations."""
    p = np.asarray(p, dtype=np.float32)
    if bias is not None:
        p = p + np.asarray(bias, dtype=np.float32)
    n = p.shape[0]
    q = p[:, :n_q * d].reshape(n, n_q, d)
    k = p[:, n_q * d:(n_q + n_kv) * d].reshape(n, n_kv, d)
    v = p[:, (n_q + n_kv) * d:].reshape(n, n_kv, d)
    q = q * (1.0 / np.sqrt(d))            # float32 * float64 scalar -> float64
    pos = np.asarray(positions, dtype=np.int64)[:, None]
    sat = 0
    if cast_after_rope:
        qi, s1 = to_fixed(rope_float(q, pos, cos, sin))
        ki, s2 = to_fixed(rope_float(k, pos, cos, sin))
        vi, s3 = to_fixed(v)
    else:
        qi, s1 = to_fixed(q)
        ki, s2 = to_fixed(k)
        vi, s3 = to_fixed(v)
        qi = rope_fixed(qi, pos, cos, sin)
        ki = rope_fixed(ki, pos, cos, sin)
    return (qi, ki, vi), s1 + s2 + s3


def fold_o_proj(o_proj, signs, n_heads: int) -> np.ndarray:
    """ops/output.py:49-78: W_o' = W_o @ blockdiag_h(R^-1) in float64, back to the input dtype."""
    w = np.asarray(o_proj)
    r = matrix(signs).T                               # R^-1 = R^T (R is orthogonal)
    d = r.shape[0]
    block = np.zeros((n_heads * d, n_heads * d), dtype=np.float64)
    for h in range(n_heads):
        block[h * d:(h + 1) * d, h * d:(h + 1) * d] = r
    return (w.astype(np.float64) @ block).astype(w.dtype)


def output_side(out_q16, w_o_folded, bias=None) -> np.ndarray:
    """kernel.py:348-356: to_float (Q16 -> float) then the W_o' projection."""
    acc = np.asarray(out_q16, dtype=np.float64) / float(1 << QK_FRAC)
    return project(w_o_folded, acc, bias)


def random_weights(hidden: int, n_q: int, n_kv: int, d: int, seed: int = 0):
    """weights.py:112-133 (the arrays before Weights.prepare's fp16 cast): q, k, v, o in
    generator order, N(0, 1) float32 times 1/sqrt(hidden) in float64."""
    rng = np.random.default_rng(seed)
    s = 1.0 / np.sqrt(hidden)

    def w(shape):
        return rng.standard_normal(shape).astype(np.float32) * s
    return (w((n_q * d, hidden)), w((n_kv * d, hidden)), w((n_kv * d, hidden)),
            w((hidden, n_q * d)))
