"""ctypes front for oracle/c/oracle.c (oracle; test infrastructure only).

Same call shapes as oracle/attention.py; used where the numpy per-token loop
would take minutes (long contexts, many steps).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from .attention import ExpLut, Stats
from .quantize import CompressedKV, Format

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")

_I64P = ctypes.POINTER(ctypes.c_int64)
_U8P = ctypes.POINTER(ctypes.c_uint8)


class _Fmt(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "d", "key_bits", "value_bits", "score_shift", "acc_shift", "prob_frac",
        "acc_frac", "score_width", "acc_width")]


class _Stats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in (
        "n_tokens", "rescale_events", "score_overflows", "acc_overflows",
        "max_abs_score", "max_abs_acc")]


class _Exp(ctypes.Structure):
    _fields_ = [("flat", ctypes.c_int64 * ((17 << 8) + 1)),
                ("delta_max", ctypes.c_int64), ("log2e", ctypes.c_int64),
                ("shift", ctypes.c_int32), ("span", ctypes.c_int32),
                ("acc_frac", ctypes.c_int32)]


def build() -> str:
    """Compile the C oracle with its committed Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        _lib = ctypes.CDLL(LIB)
    return _lib


def _p(a, t):
    return a.ctypes.data_as(t)


def _fmt(fmt: Format) -> _Fmt:
    return _Fmt(fmt.d, fmt.key_bits, fmt.value_bits, fmt.score_shift, fmt.acc_shift,
                fmt.prob_frac, fmt.acc_frac, fmt.score_width, fmt.acc_width)


def _exp(fmt: Format) -> _Exp:
    e = ExpLut(fmt)
    x = _Exp()
    tab = np.ascontiguousarray(e.table, dtype=np.int64)
    lib().orc_exp_init(ctypes.byref(x), _p(tab, _I64P), ctypes.c_int64(int(e.log2e)),
                       ctypes.c_int64(int(e.delta_max)), fmt.acc_frac, fmt.exp_lut_bits,
                       e.max_int_part)
    return x


def _stats(s: _Stats) -> Stats:
    return Stats(int(s.n_tokens), int(s.rescale_events), int(s.score_overflows),
                 int(s.acc_overflows), int(s.max_abs_score), int(s.max_abs_acc))


def _kv(kv: CompressedKV):
    return (np.ascontiguousarray(kv.k_idx, dtype=np.uint8),
            np.ascontiguousarray(kv.k_norm, dtype=np.int64),
            np.ascontiguousarray(kv.v_idx, dtype=np.uint8),
            np.ascontiguousarray(kv.v_norm, dtype=np.int64))


def exp_lut(delta, fmt: Format) -> np.ndarray:
    d = np.ascontiguousarray(delta, dtype=np.int64).reshape(-1)
    out = np.empty_like(d)
    e = _exp(fmt)
    if lib().orc_exp_vec(ctypes.byref(e), _p(d, _I64P), ctypes.c_int64(d.size), _p(out, _I64P)):
        raise ValueError("ExpLut expects a non-negative distance")
    return out.reshape(np.shape(delta))


def scores(q_rot, kv: CompressedKV, fmt: Format):
    q = np.ascontiguousarray(np.atleast_2d(q_rot), dtype=np.int64)
    ki, kn, _, _ = _kv(kv)
    T = ki.shape[0]
    s = np.empty((q.shape[0], T), dtype=np.int64)
    st = _Stats()
    f = _fmt(fmt)
    kc = np.ascontiguousarray(fmt.codebooks()[0], dtype=np.int64)
    lib().orc_scores(ctypes.byref(f), q.shape[0], _p(q, _I64P), ctypes.c_int64(T),
                     _p(ki, _U8P), _p(kn, _I64P), _p(kc, _I64P), _p(s, _I64P), ctypes.byref(st))
    return s, int(st.score_overflows)


def _attend(name: str, q_rot, kv: CompressedKV, fmt: Format, with_m: bool):
    q = np.ascontiguousarray(np.atleast_2d(q_rot), dtype=np.int64)
    G, d = q.shape
    ki, kn, vi, vn = _kv(kv)
    T = ki.shape[0]
    kc, _, vc, _ = fmt.codebooks()
    kc = np.ascontiguousarray(kc, dtype=np.int64)
    vc = np.ascontiguousarray(vc, dtype=np.int64)
    s = np.empty((G, max(T, 1)), dtype=np.int64)
    acc = np.empty((G, d), dtype=np.int64)
    l = np.empty(G, dtype=np.int64)
    m = np.empty(G, dtype=np.int64)
    out = np.empty((G, d), dtype=np.int64)
    st = _Stats()
    f = _fmt(fmt)
    e = _exp(fmt)
    args = [ctypes.byref(f), ctypes.byref(e), G, _p(q, _I64P), ctypes.c_int64(T),
            _p(ki, _U8P), _p(kn, _I64P), _p(vi, _U8P), _p(vn, _I64P),
            _p(kc, _I64P), _p(vc, _I64P), _p(s, _I64P), _p(acc, _I64P), _p(l, _I64P)]
    if with_m:
        args.append(_p(m, _I64P))
    args += [_p(out, _I64P), ctypes.byref(st)]
    getattr(lib(), name)(*args)
    return out.reshape(np.shape(q_rot)[:-1] + (d,)), _stats(st), acc, l, m


def attend_online(q_rot, kv: CompressedKV, fmt: Format):
    """Equal to oracle.attention.attend_online; returns (out, stats)."""
    out, st, _, _, _ = _attend("orc_attend_online", q_rot, kv, fmt, True)
    return out, st


def attend_online_state(q_rot, kv: CompressedKV, fmt: Format):
    """(out, stats, acc, l, m) at the end of the scan."""
    return _attend("orc_attend_online", q_rot, kv, fmt, True)


def attend_two_pass(q_rot, kv: CompressedKV, fmt: Format):
    """Equal to oracle.attention.attend_two_pass; returns (out, stats)."""
    out, st, _, _, _ = _attend("orc_attend_two_pass", q_rot, kv, fmt, False)
    return out, st


def finalize(acc, l, fmt: Format):
    acc = np.ascontiguousarray(acc, dtype=np.int64)
    l = np.ascontiguousarray(l, dtype=np.int64)
    rows, d = acc.shape
    out = np.empty_like(acc)
    r = np.empty(rows, dtype=np.int64)
    sh = np.empty(rows, dtype=np.int64)
    f = _fmt(fmt)
    lib().orc_finalize(ctypes.byref(f), rows, d, _p(acc, _I64P), _p(l, _I64P), _p(out, _I64P),
                       _p(r, _I64P), _p(sh, _I64P))
    return out, r, sh


def decode_steps(q_rot_steps, kv_heads, fmt: Format, base: int = 0) -> np.ndarray:
    """One layer's sequential decode from an empty cache, every step at once.

    q_rot_steps: (steps, n_kv * G, d) rotated query rows; kv_heads: one
    CompressedKV per KV head holding at least base + steps rows. Step i attends
    over rows 0 .. base + i (kernel.py:271-345: the token attends to itself; a
    prefill from `base`, attention.py:794-871), as attend_online does.
    Returns (steps, n_kv * G, d).
    """
    q = np.ascontiguousarray(q_rot_steps, dtype=np.int64)
    steps, rows, d = q.shape
    n_kv = len(kv_heads)
    G = rows // n_kv
    cap = kv_heads[0].k_idx.shape[0]
    ki = np.ascontiguousarray(np.stack([kv.k_idx for kv in kv_heads]), dtype=np.uint8)
    kn = np.ascontiguousarray(np.stack([kv.k_norm for kv in kv_heads]), dtype=np.int64)
    vi = np.ascontiguousarray(np.stack([kv.v_idx for kv in kv_heads]), dtype=np.uint8)
    vn = np.ascontiguousarray(np.stack([kv.v_norm for kv in kv_heads]), dtype=np.int64)
    kc, _, vc, _ = fmt.codebooks()
    kc = np.ascontiguousarray(kc, dtype=np.int64)
    vc = np.ascontiguousarray(vc, dtype=np.int64)
    out = np.empty_like(q)
    f = _fmt(fmt)
    e = _exp(fmt)
    rc = lib().orc_decode_steps(ctypes.byref(f), ctypes.byref(e), n_kv, G, ctypes.c_int64(steps),
                                ctypes.c_int64(base), ctypes.c_int64(cap), _p(q, _I64P), _p(ki, _U8P), _p(kn, _I64P),
                                _p(vi, _U8P), _p(vn, _I64P), _p(kc, _I64P), _p(vc, _I64P),
                                _p(out, _I64P))
    if rc:
        raise MemoryError("orc_decode_steps: no scratch, or base + steps > cache rows")
    return out
