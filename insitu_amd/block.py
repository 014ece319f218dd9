"""One attention block: hidden states in, hidden states out.

AttentionBlock follows the pipeline order of AttentionKernel.forward
(kernel.py:177-357 of the reference). forward() runs the host half in front
of the seam (projections, attention scale, RoPE and the fp -> fixed cast,
kernel.py:198-249, insitu_amd.host), the part below the seam, then the output
side (to_float and W_o', kernel.py:348-356). The part below the seam is:

    rotate k, v, q        kernel.py:271-276
    append k, v           kernel.py:282-284 (the current token attends to itself)
    attend per KV group   kernel.py:337-345 (query heads 4h..4h+3 share KV head h)
    merge_heads           kernel.py:352-353, ops/project.py:67-74

It is one fused C call per decode step (insitu_step), the counterpart of
the FPGA's CMD_STEP (host/attn_proto.py:65-72). A prompt of several tokens
(kernel.py:316-332) rotates and appends all its rows, then attends every
query at once (insitu_attend_causal: attend_online_batch in online mode,
attend_causal_batch in two-pass mode), bit-identical to the token loop.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .attention import AttentionStats, CompressedAttention
from .cache import CompressedCache
from .config import FixedFormat, ModelConfig, QuantConfig
from .runtime import default_context, ptr


# The chunked attend takes at most this many chunks per sequence (attend_chunked.hip, HMAX).
CHUNKED_MAX_CHUNKS = 512


def default_chunk_tokens(softmax: str, capacity: int) -> int:
    """Tokens per chunk of the chunked attend (prefill, and attends outside the decode step)
    for a block's cache. 512 for the online softmax: a model's queries (projections of
    unit-scale hidden states) give a flat softmax, whose run-sum walk 512-token chunks split
    over twice the workgroups; but only while the capacity fits the chunked attend's 512
    chunks of 512 tokens, since past that the chunked attend would refuse the cache and the
    format's attends would fall to slower kernels, while 1,024-token chunks still fit. Two-pass
    keeps 1,024 (its chunk-max launch and the prefill's query batches favour fewer chunks: a
    4,096-token two-pass prefill takes 10.1 ms on 1,024- and 17.0 ms on 512-token chunks)."""
    if softmax == "two_pass":
        return 1024
    return 512 if -(-capacity // 512) <= CHUNKED_MAX_CHUNKS else 1024


@dataclass
class StepReport:
    """kernel.py:49-67: what one forward did. `saturated` counts the fp -> fixed
    cast's clamped lanes (ConversionStats, ops/convert.py)."""

    n_tokens: int = 0
    context: int = 0
    attention: AttentionStats | None = None
    saturated: int = 0
    conversions: int = 0

    @property
    def saturation_rate(self) -> float:
        return self.saturated / self.conversions if self.conversions else 0.0

    def summary(self) -> str:
        a = self.attention or AttentionStats()
        return (f"{self.n_tokens} token(s), context {self.context}\n"
                f"  rescales {a.rescale_events}  score_ovf {a.score_overflows}  "
                f"acc_ovf {a.acc_overflows}\n"
                f"  fp->fixed saturation {self.saturation_rate:.2%}")


class AttentionBlock:
    def __init__(self, model: ModelConfig, quant: QuantConfig | None = None,
                 fmt: FixedFormat | None = None, *, capacity: int = 2048, batch: int = 1,
                 softmax: str = "online", weights=None, cast_after_rope: bool = True,
                 chunk_tokens: int | None = None, ctx=None) -> None:
        self.model = model
        self.quant = quant or QuantConfig()
        self.fmt = fmt or FixedFormat()
        self.ctx = ctx or default_context()
        if chunk_tokens is None:
            chunk_tokens = default_chunk_tokens(softmax, capacity)
        self.cache = CompressedCache(model.num_kv_heads, model.head_dim, capacity, self.quant,
                                     self.fmt, batch=batch, n_q_heads=model.num_heads,
                                     chunk_tokens=chunk_tokens, ctx=self.ctx)
        self.attn = CompressedAttention(self.cache)
        self.rotation = self.cache.rotation
        if softmax not in _lib.MODES:
            raise ValueError(f"softmax={softmax!r}; expected one of {sorted(_lib.MODES)}")
        self.softmax = softmax
        self.last_stats: AttentionStats | None = None
        # kernel.py:163: RoPE in float and one cast at the seam by default;
        # False is the board's order (cast, then fixed-point RoPE)
        self.cast_after_rope = cast_after_rope
        self.force_token_loop = False
        self.weights = weights
        self._host = None
        self.taps: dict = {}

    @property
    def batch(self) -> int:
        return self.cache.batch

    def step(self, qi, ki, vi, *, stats: bool = True):
        """One decode token per sequence.

        qi (batch, num_heads, d), ki/vi (batch, num_kv_heads, d): Q8.16 ints
        from the wire (kernel.py:256-258). Returns merge_heads(out):
        (batch, num_heads * d) Q16 in the rotated basis, as a torch int32 tensor.
        """
        import torch
        m = self.model
        q = self.ctx.to_device(qi, torch.int32).reshape(self.batch, m.num_heads, m.head_dim)
        k = self.ctx.to_device(ki, torch.int32).reshape(self.batch, m.num_kv_heads, m.head_dim)
        v = self.ctx.to_device(vi, torch.int32).reshape(self.batch, m.num_kv_heads, m.head_dim)
        out = torch.empty_like(q)
        st = _lib.Stats() if stats else None
        _lib.check(self.ctx.lib.insitu_step(self.cache.handle, ptr(q), ptr(k), ptr(v), ptr(out),
                                            _lib.MODES[self.softmax],
                                            ctypes.byref(st) if st is not None else None))
        self._keep = (q, k, v)
        self.last_stats = AttentionStats.from_c(st) if st is not None else None
        return out.reshape(self.batch, m.num_heads * m.head_dim)

    def prefill(self, qi, ki, vi, *, stats: bool = True):
        """batch == 1, a prompt of n tokens: qi (n, num_heads, d), ki/vi
        (n, num_kv_heads, d) wire Q8.16. Rotates all three, appends the n rows,
        then query t attends rows 0 .. base + t (kernel.py:316-332). Returns
        (n, num_heads * d) Q16, a torch int32 tensor."""
        import torch
        m = self.model
        if self.batch != 1:
            raise ValueError("prefill drives a batch-1 block")
        q = self.ctx.to_device(qi, torch.int32)
        n = int(q.shape[0])
        q = q.reshape(n, m.num_heads, m.head_dim)
        k = self.ctx.to_device(ki, torch.int32).reshape(n, m.num_kv_heads, m.head_dim)
        v = self.ctx.to_device(vi, torch.int32).reshape(n, m.num_kv_heads, m.head_dim)
        base = self.cache.length
        qr = self.rotation.apply(q, self.ctx)
        self.cache.append_wire(k, v)            # rotate and append in one launch
        out, st = self.attn.attend_prefill(qr, base, self.softmax, stats=stats)
        self.last_stats = st
        return out.reshape(n, m.num_heads * m.head_dim)

    def forward_seam(self, qi, ki, vi, *, force_token_loop: bool = False) -> np.ndarray:
        """batch == 1: (tokens, heads, d) wire tensors.

        Several tokens go through prefill (kernel.py:316-332), one token (or
        force_token_loop, kernel.py:333-341) through decode steps. Returns
        (tokens, num_heads * d) int64, the `out` tap of kernel.py:353.
        """
        qi, ki, vi = (np.asarray(a) for a in (qi, ki, vi))
        if self.batch != 1:
            raise ValueError("forward_seam drives a batch-1 block")
        if qi.shape[0] > 1 and not force_token_loop:
            return self.prefill(qi, ki, vi).cpu().numpy().astype(np.int64)
        outs = [self.step(qi[t][None], ki[t][None], vi[t][None]).cpu().numpy()
                for t in range(qi.shape[0])]
        return np.concatenate(outs, axis=0).astype(np.int64)

    @property
    def host(self):
        if self.weights is None:
            raise ValueError("forward needs weights: AttentionBlock(..., weights=Weights(...))")
        if self._host is None or self._host.cast_after_rope != self.cast_after_rope:
            from .host import HostHalf
            self._host = HostHalf(self.model, self.weights, cast_after_rope=self.cast_after_rope,
                                  ctx=self.ctx)
        return self._host

    def forward(self, hidden_states, positions=None, *, stats: bool = True):
        """kernel.py:177-357, batch == 1: (tokens, hidden) float32 in, (tokens,
        hidden) float32 out (a torch tensor on the device), and a StepReport.

        positions default to cache.length .. cache.length + tokens - 1. The
        wire rows and the Q16 `out` rows are kept in self.taps ("wire.q",
        "wire.k", "wire.v", "out"), the reference's tap points. stats=False
        leaves the report's counters empty and the step stream-ordered (the
        counters are the only values read back before the output).
        """
        import torch
        m = self.model
        if self.batch != 1:
            raise ValueError("forward drives a batch-1 block")
        x = self.ctx.to_device(hidden_states, torch.float32)
        if x.dim() == 1:
            x = x[None, :]
        if x.shape[-1] != m.hidden_size:
            raise ValueError(f"hidden size {x.shape[-1]} != {m.hidden_size}")
        n = int(x.shape[0])
        base = self.cache.length
        if positions is None:
            positions = np.arange(base, base + n)
        positions = np.asarray(positions, dtype=np.int64)
        if positions.shape != (n,):
            raise ValueError(f"expected {n} positions, got {positions.shape}")
        host = self.host
        qi, ki, vi = host.wire(x, positions, counts=stats)
        self.taps = {"wire.q": qi, "wire.k": ki, "wire.v": vi}
        report = StepReport(n_tokens=n)
        if stats:
            report.saturated = host.last_saturated
            report.conversions = n * (m.num_heads + 2 * m.num_kv_heads) * m.head_dim
        if n > 1 and not self.force_token_loop:
            out = self.prefill(qi, ki, vi, stats=stats)
            report.attention = self.last_stats
        else:
            rows = []
            report.attention = AttentionStats() if stats else None
            for t in range(n):
                rows.append(self.step(qi[t][None], ki[t][None], vi[t][None], stats=stats))
                if stats:
                    report.attention.merge(self.last_stats)
            out = rows[0] if n == 1 else torch.cat(rows, dim=0)
        self.taps["out"] = out
        report.context = base + n
        return host.output(out), report

    def reset(self) -> None:
        """kernel.py:454-456: a new sequence; tables survive."""
        self.cache.reset()
