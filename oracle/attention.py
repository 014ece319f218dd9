"""Scores on codes, exp LUT, online / two-pass softmax, reciprocal and finalize.

Oracle; test infrastructure only. Restates ops/attention.py:90-513 and :873-880
of the reference, plus the qtab definition of hw/vectors.py:485-509.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .fixed import I64, Q, rshift
from .quantize import CompressedKV, Format

L_WIDTH = 48                 # attention.py:174
RECIP_NORM_BITS = 32         # attention.py:193
RECIP_NUM_SHIFT = 62         # attention.py:194


class ExpLut:
    """exp(-x) as 2^-i * 2^-f; attention.py:90-169."""

    def __init__(self, fmt: Format) -> None:
        self.fmt = fmt
        n = 1 << fmt.exp_lut_bits
        frac = np.arange(n, dtype=np.float64) / n
        self.table = np.rint(2.0 ** (-frac) * (1 << fmt.prob_frac)).astype(I64)
        self.log2e = I64(round(np.log2(np.e) * (1 << fmt.acc_frac)))
        self.max_int_part = fmt.prob_frac + 1
        self.shift = fmt.acc_frac - fmt.exp_lut_bits
        span = (self.max_int_part + 1) << fmt.exp_lut_bits
        self.span = span
        # attention.py:145-146: smallest delta whose flat index reaches `span`.
        self.delta_max = I64(-(-((span << self.shift) << fmt.acc_frac) // int(self.log2e)))
        u = np.arange(span, dtype=I64)
        flat = self.table[u & (n - 1)] >> np.minimum(u >> fmt.exp_lut_bits, self.max_int_part)
        flat[(u >> fmt.exp_lut_bits) > self.max_int_part] = 0
        self.flat = np.concatenate([flat, np.zeros(1, dtype=I64)])

    def __call__(self, delta) -> np.ndarray:
        """attention.py:153-159: round(2^15 exp(-delta / 2^16)), delta >= 0."""
        d = np.minimum(np.asarray(delta, dtype=I64), self.delta_max)
        if np.any(d < 0):
            raise ValueError("ExpLut expects a non-negative distance below the running max")
        t = rshift(d * self.log2e, self.fmt.acc_frac)
        return self.flat[np.minimum(t >> I64(self.shift), self.span)]

    def two_step(self, delta) -> np.ndarray:
        """attention.py:161-169: table read plus a shift."""
        d = np.minimum(np.asarray(delta, dtype=I64), self.delta_max)
        t = rshift(d * self.log2e, self.fmt.acc_frac)
        i = rshift(t, self.fmt.acc_frac)
        f = t & ((I64(1) << I64(self.fmt.acc_frac)) - 1)
        addr = rshift(f, self.fmt.acc_frac - self.fmt.exp_lut_bits)
        p = self.table[addr] >> np.minimum(i, self.max_int_part)
        return np.where(i > self.max_int_part, I64(0), p)


def lead(l) -> np.ndarray:
    """attention.py:177-183: leading-one position, capped at L_WIDTH-1, 0 for 0 and 1."""
    a = np.asarray(l, dtype=I64)
    n = np.zeros_like(a)
    for b in range(1, L_WIDTH):
        n = np.where(a >= (I64(1) << I64(b)), I64(b), n)
    return n


def reciprocal(l, fmt: Format):
    """attention.py:197-250: (recip, shift) with out = (acc * recip) >> shift."""
    a = np.asarray(l, dtype=I64)
    s = lead(a)
    k = s - (RECIP_NORM_BITS - 1)
    l_n = np.where(k >= 0, a >> np.maximum(k, 0), a << np.maximum(-k, 0))
    num = I64(1) << I64(RECIP_NUM_SHIFT)
    r = np.where(a > 0, num // np.maximum(l_n, I64(1)), I64(0))
    return r, RECIP_NUM_SHIFT - fmt.prob_frac + k


def finalize(acc, l, fmt: Format) -> np.ndarray:
    """attention.py:873-880."""
    r, sh = reciprocal(l, fmt)
    return rshift(np.asarray(acc, dtype=I64) * r[..., None], sh[..., None])


@dataclass
class Stats:
    """attention.py:257-274."""

    n_tokens: int = 0
    rescale_events: int = 0
    score_overflows: int = 0
    acc_overflows: int = 0
    max_abs_score: int = 0
    max_abs_acc: int = 0

    def merge(self, o: "Stats") -> None:
        self.n_tokens = max(self.n_tokens, o.n_tokens)
        self.rescale_events += o.rescale_events
        self.score_overflows += o.score_overflows
        self.acc_overflows += o.acc_overflows
        self.max_abs_score = max(self.max_abs_score, o.max_abs_score)
        self.max_abs_acc = max(self.max_abs_acc, o.max_abs_acc)


def qtab(q_rot, key_centroids) -> np.ndarray:
    """hw/vectors.py:485-509 (== the einsum of attention.py:344-352): T[h, ch, i] = q[h, ch] * c[i]."""
    return np.asarray(q_rot, dtype=I64)[..., :, None] * np.asarray(key_centroids, dtype=I64)


def scores(q_rot, kv: CompressedKV, fmt: Format):
    """attention.py:333-359: clamp48(floor((sum_ch q * c[code]) * k_norm / 2^24)).

    Returns (scores, overflow_count). int64 arithmetic wraps exactly as numpy does.
    """
    kc = fmt.codebooks()[0]
    codes = kc[np.asarray(kv.k_idx, dtype=I64)]
    q = np.asarray(q_rot, dtype=I64)
    dot = np.einsum("...j,tj->...t", q, codes)
    s = rshift(dot * np.asarray(kv.k_norm, dtype=I64), fmt.score_shift)
    sq = Q(fmt.score_width, fmt.acc_frac)
    return sq.clamp(s), sq.overflow_count(s)


def accumulate_terms(p, kv: CompressedKV, fmt: Format) -> np.ndarray:
    """attention.py:400-425 (fused branch): floor(v_norm * p * c_v[code] / 2^acc_shift) per term."""
    vc = fmt.codebooks()[2]
    v_hat = vc[np.asarray(kv.v_idx, dtype=I64)]
    weight = np.asarray(kv.v_norm, dtype=I64)[..., None] * np.asarray(p, dtype=I64)[..., None]
    return rshift(weight * v_hat, fmt.acc_shift)


def attend_two_pass(q_rot, kv: CompressedKV, fmt: Format):
    """attention.py:429-449: global max, one accumulation, clamp at the end."""
    exp = ExpLut(fmt)
    s, ovf = scores(q_rot, kv, fmt)
    st = Stats(n_tokens=s.shape[-1], score_overflows=ovf,
               max_abs_score=int(np.abs(s).max(initial=0)))
    m = s.max(axis=-1, keepdims=True)
    p = exp(m - s)
    l = p.sum(axis=-1)
    acc = accumulate_terms(p, kv, fmt).sum(axis=-2)
    aq = Q(fmt.acc_width, fmt.acc_frac)
    st.acc_overflows = aq.overflow_count(acc)
    acc = aq.clamp(acc)
    st.max_abs_acc = int(np.abs(acc).max(initial=0))
    return finalize(acc, l, fmt), st


def attend_online(q_rot, kv: CompressedKV, fmt: Format, on_step=None):
    """attention.py:451-513: the sequential-order golden.

    Per token t: if s_t > m, rescale acc and l by f = LUT(s_t - m) (floor), m = s_t;
    p = LUT(m - s_t); l += p; acc += floor(v_norm p c_v[code] / 2^acc_shift);
    clamp acc to int32 every token. `on_step(t, s, m, p, l, acc, grew, factor)`
    observes copies, like attention.py:505-507.
    """
    exp = ExpLut(fmt)
    s, ovf = scores(q_rot, kv, fmt)
    s = np.atleast_2d(s)
    n_heads, n_tok = s.shape
    st = Stats(n_tokens=n_tok, score_overflows=ovf,
               max_abs_score=int(np.abs(s).max(initial=0)))
    d = fmt.d
    aq = Q(fmt.acc_width, fmt.acc_frac)
    sq = Q(fmt.score_width, fmt.acc_frac)
    acc = np.zeros((n_heads, d), dtype=I64)
    l = np.zeros(n_heads, dtype=I64)
    m = np.full(n_heads, sq.lo, dtype=I64)
    unity = I64(1) << I64(fmt.prob_frac)
    vc = fmt.codebooks()[2]
    for t in range(n_tok):
        stt = s[:, t]
        grew = stt > m
        factor = None
        if grew.any():
            delta = np.where(grew, stt - m, 0)
            factor = np.where(grew, exp(delta), unity)
            acc = rshift(acc * factor[:, None], fmt.prob_frac)
            l = rshift(l * factor, fmt.prob_frac)
            m = np.where(grew, stt, m)
            st.rescale_events += int(grew.sum())
        p = exp(m - stt)
        l = l + p
        v_hat = vc[np.asarray(kv.v_idx[t], dtype=I64)]
        acc = acc + rshift((I64(kv.v_norm[t]) * p)[:, None] * v_hat, fmt.acc_shift)
        st.acc_overflows += aq.overflow_count(acc)
        acc = aq.clamp(acc)
        if on_step is not None:
            on_step(t, s=stt.copy(), m=m.copy(), p=p.copy(), l=l.copy(), acc=acc.copy(),
                    grew=grew.copy(), factor=None if factor is None else factor.copy())
    st.max_abs_acc = int(np.abs(acc).max(initial=0))
    out = finalize(acc, l, fmt)
    return out.reshape(np.shape(q_rot)[:-1] + (d,)), st


def attend_online_state(q_rot, kv: CompressedKV, fmt: Format):
    """attend_online without the finalize: (acc, l, m) at the end of the scan."""
    box = {}

    def grab(t, **kw):
        box.update(kw)

    attend_online(q_rot, kv, fmt, on_step=grab)
    return box.get("acc"), box.get("l"), box.get("m")
