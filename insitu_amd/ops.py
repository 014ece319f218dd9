"""Single-stage device entry points, for stage-by-stage parity with the reference.

Each runs one block of the path on the GPU and returns host numpy arrays:

    encode     KVQuantizer._norm_wire + _encode_plane   ops/quantize.py:164-196
    qtab       T[h][ch][i] = q_rot[h][ch] * c[i]        hw/vectors.py:485-509
    exp_lut    ExpLut.__call__                          ops/attention.py:153-159
    finalize   reciprocal + _finalize                   ops/attention.py:197-250, 873-880
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .runtime import default_context, i64p, ptr


def encode(x_rot, boundaries, bits: int, *, d: int | None = None, norm_frac: int = 9, ctx=None):
    """(n, d) rotated Q16 ints -> (norms (n,) int64, codes (n, d) uint8)."""
    import torch
    ctx = ctx or default_context()
    x = ctx.to_device(x_rot, torch.int32)
    n, dd = x.shape
    f = _lib.Format()
    f.head_dim = d or dd
    f.key_bits = f.value_bits = bits
    f.norm_bits, f.norm_frac = 16, norm_frac
    f.qk_frac, f.qk_width, f.centroid_frac = 16, 24, 15
    f.acc_frac, f.acc_width, f.score_width = 16, 32, 48
    f.prob_frac, f.exp_lut_bits, f.rot_rounds = 15, 8, 1
    b = np.ascontiguousarray(boundaries, dtype=np.int64)
    if b.shape != ((1 << bits) - 1,):
        raise ValueError("boundaries must have 2**bits - 1 entries")
    norm = torch.empty(n, dtype=torch.int32, device=x.device)
    codes = torch.empty((n, dd), dtype=torch.uint8, device=x.device)
    _lib.check(ctx.lib.insitu_encode(ctx.handle, ptr(x), n, ctypes.byref(f), i64p(b), bits,
                                     ptr(norm), ptr(codes)))
    return norm.cpu().numpy().astype(np.int64), codes.cpu().numpy()


def qtab(q_rot, centroids, ctx=None) -> np.ndarray:
    """(heads, d) rotated queries -> (heads, d, n_centroids) int64 products."""
    import torch
    ctx = ctx or default_context()
    q = ctx.to_device(q_rot, torch.int32)
    h, d = q.shape
    c = np.ascontiguousarray(centroids, dtype=np.int64)
    out = torch.empty((h, d, c.size), dtype=torch.int64, device=q.device)
    _lib.check(ctx.lib.insitu_qtab(ctx.handle, ptr(q), h, d, i64p(c), c.size, ptr(out)))
    return out.cpu().numpy()


def exp_lut(delta, ctx=None) -> np.ndarray:
    """round(2^15 exp(-delta / 2^16)) for delta >= 0; raises on a negative delta like ExpLut."""
    import torch
    ctx = ctx or default_context()
    dl = np.asarray(delta, dtype=np.int64)
    if np.any(dl < 0):
        raise ValueError("ExpLut expects a non-negative distance below the running max")
    d = ctx.to_device(dl.reshape(-1), torch.int64)
    p = torch.empty(d.numel(), dtype=torch.int32, device=d.device)
    _lib.check(ctx.lib.insitu_exp_lut(ctx.handle, ptr(d), d.numel(), ptr(p)))
    return p.cpu().numpy().astype(np.int64).reshape(dl.shape)


def finalize(acc, l, ctx=None):
    """(rows, d) accumulators and (rows,) denominators -> (out, recip, shift)."""
    import torch
    ctx = ctx or default_context()
    a = ctx.to_device(np.asarray(acc, dtype=np.int64), torch.int64)
    lv = ctx.to_device(np.asarray(l, dtype=np.int64), torch.int64)
    rows, d = a.shape
    out = torch.empty_like(a)
    r = torch.empty(rows, dtype=torch.int64, device=a.device)
    sh = torch.empty(rows, dtype=torch.int32, device=a.device)
    _lib.check(ctx.lib.insitu_finalize(ctx.handle, ptr(a), ptr(lv), rows, d, ptr(out), ptr(r),
                                       ptr(sh)))
    return out.cpu().numpy(), r.cpu().numpy(), sh.cpu().numpy().astype(np.int64)
