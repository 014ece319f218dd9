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


def fill_ragged(cache, lens, seed: int, rot, ctx, keep=()):
    """C3's data: sequence b of `cache` gets lens[b] tokens of k/v and one query row per
    head from Workload(seed=seed + b) (the four-outlier distribution), k/v rotated on
    the device and appended. Returns (q_rot (batch, n_q, d) int64, {b: (k_rot, v_rot)}
    for the sequences in `keep`, as int64 host arrays)."""
    d, n_kv, n_q = cache.head_dim, cache.n_kv_heads, cache.n_q_heads
    q = np.zeros((cache.batch, n_q, d), dtype=np.int64)
    kept = {}
    for b, n in enumerate(lens):
        wl = Workload(n_q_heads=n_q, n_kv_heads=n_kv, head_dim=d, seed=seed + b)
        n = int(n)
        kw = wl.rng.standard_normal((n, n_kv, d), dtype=np.float32) * wl.k_scale
        vw = wl.rng.standard_normal((n, n_kv, d), dtype=np.float32) * wl.v_scale
        qw = wl.rng.standard_normal((n_q, d), dtype=np.float32) * wl.q_scale
        kr = rot.apply(to_fixed(kw), ctx)
        vr = rot.apply(to_fixed(vw), ctx)
        if n:
            cache.append_rotated(kr, vr, seq=b)
        q[b] = rot.apply(to_fixed(qw), ctx).cpu().numpy()
        if b in keep:
            kept[b] = (kr.cpu().numpy().astype(np.int64), vr.cpu().numpy().astype(np.int64))
    return q, kept


def _device_fixed(gen, shape, scale, ctx):
    """N(0,1) float32 on the device times per-head channel scales, cast to Q8.16 (rint,
    24-bit saturation): to_fixed of the same distribution."""
    import torch
    x = torch.randn(shape, generator=gen, device=ctx.torch_device, dtype=torch.float32) * scale
    x = torch.round(x.double() * float(1 << QK_FRAC))
    return x.clamp_(-(1 << (QK_WIDTH - 1)), (1 << (QK_WIDTH - 1)) - 1).to(torch.int32)


def fill_on_device(cache, n_tokens: int, seed: int, rot, ctx, *, outlier_p: float = 0.01,
                   outlier_scale: float = 16.0, block: int = 16384, sample_rows: int = 0):
    """C4's data, drawn on the GPU (numpy would take minutes for 2 G values): every
    sequence b gets n_tokens of k/v from a torch.Generator seeded seed + b, N(0,1) with
    each channel of each head an outlier (x outlier_scale) with probability outlier_p
    (the mask from numpy default_rng(seed + b)), cast to Q8.16, rotated and appended in
    blocks. The queries (one row per head per sequence) come from seed + batch.
    Returns (q_rot (batch, n_q, d) int64, {b: (rows, k_rot, v_rot)}: sample_rows rows of
    one block of each sequence, for checking the encoder)."""
    import torch
    d, n_kv, n_q, batch = cache.head_dim, cache.n_kv_heads, cache.n_q_heads, cache.batch
    dev = ctx.torch_device

    def scales(rng, heads):
        m = np.where(rng.random((heads, d)) < outlier_p, outlier_scale, 1.0).astype(np.float32)
        return torch.from_numpy(m).to(dev)

    samples = {}
    pick_rng = np.random.default_rng(seed)
    for b in range(batch):
        gen = torch.Generator(device=dev).manual_seed(seed + b)
        srng = np.random.default_rng(seed + b)
        ks, vs = scales(srng, n_kv), scales(srng, n_kv)
        sample_at = (b % max(1, n_tokens // block)) * block
        for t0 in range(0, n_tokens, block):
            n = min(block, n_tokens - t0)
            kr = rot.apply(_device_fixed(gen, (n, n_kv, d), ks, ctx).reshape(-1, d), ctx).reshape(n, n_kv, d)
            vr = rot.apply(_device_fixed(gen, (n, n_kv, d), vs, ctx).reshape(-1, d), ctx).reshape(n, n_kv, d)
            cache.append_rotated(kr, vr, seq=b)
            if sample_rows and t0 == sample_at:
                pick = np.sort(pick_rng.choice(n, min(sample_rows, n), replace=False))
                samples[b] = (t0 + pick, kr[pick].cpu().numpy().astype(np.int64),
                              vr[pick].cpu().numpy().astype(np.int64))
    qgen = torch.Generator(device=dev).manual_seed(seed + batch)
    qs = scales(np.random.default_rng(seed + batch), n_q)
    qw = _device_fixed(qgen, (batch, n_q, d), qs, ctx)
    q = rot.apply(qw.reshape(-1, d), ctx).reshape(batch, n_q, d).cpu().numpy().astype(np.int64)
    return q, samples
