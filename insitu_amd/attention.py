"""Attention on the codes, on the GPU.

CompressedAttention mirrors ops/attention.py:281-513 of the reference: the
same two softmaxes (`attend_online`, the hardware's sequential order, and
`attend_two_pass`) and the same AttentionStats, computed by libinsitu_hip.so
over an HBM-resident CompressedCache. Query heads that share a KV head are
attended together (kernel.py:303-345).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from .cache import CompressedCache, DeviceKV
from .runtime import ptr


@dataclass
class AttentionStats:
    """attention.py:257-274, plus the device's range/fallback counters."""

    n_tokens: int = 0
    rescale_events: int = 0
    score_overflows: int = 0
    acc_overflows: int = 0
    max_abs_score: int = 0
    max_abs_acc: int = 0
    range_errors: int = 0
    serial_fallbacks: int = 0

    def merge(self, other: "AttentionStats") -> None:
        self.n_tokens = max(self.n_tokens, other.n_tokens)
        self.rescale_events += other.rescale_events
        self.score_overflows += other.score_overflows
        self.acc_overflows += other.acc_overflows
        self.max_abs_score = max(self.max_abs_score, other.max_abs_score)
        self.max_abs_acc = max(self.max_abs_acc, other.max_abs_acc)
        self.range_errors += other.range_errors
        self.serial_fallbacks += other.serial_fallbacks

    @classmethod
    def from_c(cls, s: "_lib.Stats") -> "AttentionStats":
        return cls(*(int(getattr(s, n)) for n, _ in _lib.Stats._fields_))


def _shape(a) -> tuple:
    return tuple(a.shape) if hasattr(a, "shape") else np.shape(a)


class CompressedAttention:
    """Scores and accumulates on codes for every sequence and KV head of a cache."""

    def __init__(self, cache: CompressedCache) -> None:
        self.cache = cache
        self.ctx = cache.ctx

    def attend(self, q_rot, mode: str = "online", out=None, stats: bool = True):
        """q_rot (batch, n_q_heads, d) rotated Q8.16 -> out (batch, n_q_heads, d) Q16.

        mode: "online" (attend_online, bit-exact), "two_pass" (attend_two_pass,
        bit-exact), "split" (context-split), "serial" (one token at a time).
        Returns (out torch int32 tensor, AttentionStats or None). With
        stats=False nothing synchronises.
        """
        import torch
        c = self.cache
        q = self.ctx.to_device(q_rot, torch.int32)
        if q.dim() == 2 and c.batch == 1:
            q = q.unsqueeze(0)
        if q.shape != (c.batch, c.n_q_heads, c.head_dim):
            raise ValueError(f"q_rot must be ({c.batch}, {c.n_q_heads}, {c.head_dim}), "
                             f"got {tuple(q.shape)}")
        if out is None:
            out = torch.empty_like(q)
        st = _lib.Stats() if stats else None
        _lib.check(self.ctx.lib.insitu_attend(c.handle, ptr(q), ptr(out), _lib.MODES[mode],
                                              ctypes.byref(st) if st is not None else None))
        self._keep = q
        return out, (AttentionStats.from_c(st) if st is not None else None)

    # -- one KV head: the reference's call forms (kernel.py:317-331, 385-392) --------

    score_mode = "fused"     # attention.py:323: scores on the codes (architecture B)

    def _kv(self, kv, seq: int) -> DeviceKV:
        if isinstance(kv, (int, np.integer)):
            return self.cache.view(int(kv), seq=seq)
        if not isinstance(kv, DeviceKV) or kv.cache is not self.cache:
            raise TypeError("kv must be this cache's view (CompressedCache.view) or a KV head index")
        return kv

    def _head(self, q_rot, kv: DeviceKV, base: int, n_q: int, mode: str):
        import torch
        c = self.cache
        g = c.n_q_heads // c.n_kv_heads
        q = self.ctx.to_device(q_rot, torch.int32)
        if q.numel() != n_q * g * c.head_dim:
            raise ValueError(f"expected {n_q} x {g} query heads of {c.head_dim} for one KV group, "
                             f"got {tuple(q.shape)}")
        if base < 0 or base + n_q > kv.stop:
            raise ValueError(f"queries {base} .. {base + n_q - 1} attend rows 0 .. base + i, "
                             f"but the view holds {kv.stop} rows")
        q = q.reshape(n_q, g, c.head_dim).contiguous()
        out = torch.empty_like(q)
        st = _lib.Stats()
        _lib.check(self.ctx.lib.insitu_attend_causal_head(c.handle, kv.seq, kv.kv_head, base, n_q, ptr(q),
                                                          ptr(out), _lib.MODES[mode], ctypes.byref(st)))
        res = out.cpu().numpy().astype(np.int64)
        return res.reshape(_shape(q_rot)[:-1] + (c.head_dim,)), AttentionStats.from_c(st)

    def attend_online(self, q_rot, kv, trace=None, *, seq: int = 0):
        """attention.py:451-513: the G query heads of one KV head (q_rot (G, d) or (d,))
        against every row of `kv` -> (out int64 of q_rot's shape, AttentionStats).
        kv: this cache's view of the head (cache.view(h).select(slice(0, ctx)), the
        call of kernel.py:385-392), or the KV head's index (all its rows, sequence
        `seq`). trace is accepted for the reference's call form and left untouched."""
        kv = self._kv(kv, seq)
        return self._head(q_rot, kv, kv.stop - 1, 1, "online")

    def attend_two_pass(self, q_rot, kv, trace=None, *, seq: int = 0):
        """attention.py:429-449, the same call form."""
        kv = self._kv(kv, seq)
        return self._head(q_rot, kv, kv.stop - 1, 1, "two_pass")

    # -- prefill: every query of a prompt at once (attention.py:517-871) --------

    def attend_prefill(self, q_rot, base: int = 0, mode: str = "online", seq: int = 0, out=None,
                       stats: bool = True):
        """q_rot (n_q, n_q_heads, d) rotated: query i attends rows 0 .. base + i of
        sequence `seq` (its own row included; the prompt's rows are appended
        first). mode "online" is attend_online_batch (attention.py:794-871),
        "two_pass" attend_causal_batch (:517-670), "serial" the token loop.
        Returns (out torch int32 (n_q, n_q_heads, d), AttentionStats or None)."""
        import torch
        c = self.cache
        q = self.ctx.to_device(q_rot, torch.int32)
        if q.dim() != 3 or q.shape[1:] != (c.n_q_heads, c.head_dim):
            raise ValueError(f"q_rot must be (n_q, {c.n_q_heads}, {c.head_dim}), got {tuple(q.shape)}")
        q = q.contiguous()
        if out is None:
            out = torch.empty_like(q)
        st = _lib.Stats() if stats else None
        _lib.check(self.ctx.lib.insitu_attend_causal(c.handle, seq, base, q.shape[0], ptr(q), ptr(out),
                                                     _lib.MODES[mode],
                                                     ctypes.byref(st) if st is not None else None))
        self._keep = q
        return out, (AttentionStats.from_c(st) if st is not None else None)

    def attend_causal_batch(self, q_rot, kv, base: int = 0, tile: int = 256, trace=None, *, seq: int = 0):
        """attention.py:517-670 for one KV head, the call of kernel.py:329-331:
        q_rot (n_q, G, d); query i attends rows 0 .. base + i of kv by
        attend_two_pass. tile is the reference's memory bound on its float64
        evaluation and changes nothing here. -> (out (n_q, G, d) int64, stats)."""
        kv = self._kv(kv, seq)
        return self._head(q_rot, kv, base, int(_shape(q_rot)[0]), "two_pass")

    def attend_online_batch(self, q_rot, kv, base: int = 0, trace=None, *, seq: int = 0):
        """attention.py:794-871 for one KV head (kernel.py:326-327), by attend_online."""
        kv = self._kv(kv, seq)
        return self._head(q_rot, kv, base, int(_shape(q_rot)[0]), "online")
