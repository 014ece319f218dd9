"""The host half of the block on the GPU: the projections, RoPE and the cast in
front of the seam, and the output projection behind it.

Mirrors the reference's weights.py (Weights.prepare / random, :32-133),
ops/rope.py (RopeScaling, RoPE.build, :48-142) and the parts of
AttentionKernel.forward (kernel.py:198-249, 348-356) that run on the host.
The tables and the weight fold are built once on the host in float64, as the
reference builds them; every per-token step runs in libinsitu_hip.so
(insitu_project, insitu_seam_wire, insitu_output_projection).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from .runtime import default_context, ptr

ROPE_FRAC = 15          # config.py:225: the sin/cos table is Q1.15, as the codebooks are


@dataclass(frozen=True)
class RopeScaling:
    """ops/rope.py:48-115: Llama 3's frequency rescaling, applied to inv_freq."""

    factor: float
    low_freq_factor: float
    high_freq_factor: float
    original_max_position: int

    def __post_init__(self) -> None:
        if not self.high_freq_factor > self.low_freq_factor:
            raise ValueError(f"high_freq_factor={self.high_freq_factor} must exceed "
                             f"low_freq_factor={self.low_freq_factor}")

    @classmethod
    def from_hf(cls, params: dict) -> "RopeScaling":
        return cls(float(params["factor"]), float(params["low_freq_factor"]),
                   float(params["high_freq_factor"]), int(params["original_max_position_embeddings"]))

    def apply(self, inv_freq) -> np.ndarray:
        f = np.asarray(inv_freq, dtype=np.float64)
        ctx = float(self.original_max_position)
        wavelen = 2.0 * np.pi / f
        low_w = ctx / self.low_freq_factor
        high_w = ctx / self.high_freq_factor
        scaled = np.where(wavelen > low_w, f / self.factor, f)
        smooth = (ctx / wavelen - self.low_freq_factor) / (self.high_freq_factor - self.low_freq_factor)
        mid = (1.0 - smooth) * scaled / self.factor + smooth * scaled
        return np.where((wavelen <= low_w) & (wavelen >= high_w), mid, scaled)


@dataclass(frozen=True)
class RoPE:
    """ops/rope.py:117-142: cos/sin for every reachable position, Q(32, frac), built
    once in float64 (half to even); held on the device as int64 (max_position, d/2)."""

    cos: np.ndarray
    sin: np.ndarray
    frac: int

    @staticmethod
    def build(d: int, max_position: int, theta: float = 10000.0, frac: int = ROPE_FRAC,
              scaling: RopeScaling | None = None) -> "RoPE":
        if d % 2:
            raise ValueError(f"head_dim={d} must be even: RoPE rotates channel pairs")
        half = d // 2
        inv = 1.0 / (theta ** (np.arange(0, half, dtype=np.float64) * 2.0 / d))
        if scaling is not None:
            inv = scaling.apply(inv)
        ang = np.arange(max_position, dtype=np.float64)[:, None] * inv[None, :]

        def q(a):
            return np.clip(np.rint(a * float(1 << frac)), -(1 << 31), (1 << 31) - 1).astype(np.int64)
        return RoPE(q(np.cos(ang)), q(np.sin(ang)), frac)


def fold_o_proj(o_proj, rotation_matrix: np.ndarray, num_heads: int) -> np.ndarray:
    """ops/output.py:49-78: W_o' = W_o @ blockdiag_h(R^-1), in float64."""
    w = np.asarray(o_proj, dtype=np.float64)
    r = np.asarray(rotation_matrix, dtype=np.float64).T      # R^-1 acting on a row
    d = r.shape[0]
    if w.shape[1] != num_heads * d:
        raise ValueError(f"o_proj takes {w.shape[1]} input channels, the block produces "
                         f"{num_heads} x {d}")
    out = np.empty_like(w)
    for h in range(num_heads):
        out[:, h * d:(h + 1) * d] = w[:, h * d:(h + 1) * d] @ r
    return out


def _host_array(a):
    """A checkpoint tensor (torch, on any device, with or without grad) or array -> numpy."""
    if a is None or isinstance(a, np.ndarray):
        return a
    if hasattr(a, "detach"):
        return a.detach().float().cpu().numpy()
    return np.asarray(a)


class Weights:
    """weights.py:32-133: fp16 W_q | W_k | W_v stacked (the checkpoint's (out, in) layout),
    fp16 W_o' (R^-1 folded), fp32 biases; device-resident. rotation_matrix is the
    cache's Rotation or its dense matrix (R_last ... R_0)."""

    def __init__(self, q, k, v, o, model, rotation_matrix, *, q_bias=None, k_bias=None,
                 v_bias=None, o_bias=None, ctx=None) -> None:
        import torch
        self.model = model
        self.ctx = ctx or default_context()
        q, k, v, o, q_bias, k_bias, v_bias, o_bias = (
            _host_array(a) for a in (q, k, v, o, q_bias, k_bias, v_bias, o_bias))
        shapes = {"q": (model.q_out_features, model.hidden_size),
                  "k": (model.kv_out_features, model.hidden_size),
                  "v": (model.kv_out_features, model.hidden_size),
                  "o": (model.hidden_size, model.q_out_features)}
        for name, arr in (("q", q), ("k", k), ("v", v), ("o", o)):
            if np.shape(arr) != shapes[name]:
                raise ValueError(f"W_{name} is {np.shape(arr)}, expected {shapes[name]}")
        f16 = lambda a: np.asarray(a, dtype=np.float16)
        qkv = np.concatenate([f16(q), f16(k), f16(v)])
        if hasattr(rotation_matrix, "matrix"):              # a Rotation
            rotation_matrix = rotation_matrix.matrix()
        o_folded = f16(fold_o_proj(o, rotation_matrix, model.num_heads))
        dev = self.ctx.torch_device
        self.qkv = torch.from_numpy(qkv.view(np.int16)).to(dev)
        self.o = torch.from_numpy(o_folded.view(np.int16)).to(dev)
        biases = [q_bias, k_bias, v_bias]
        if any(b is not None for b in biases):
            full = np.concatenate([np.zeros(n, np.float32) if b is None else np.asarray(b, np.float32)
                                   for b, n in zip(biases, (shapes["q"][0], shapes["k"][0], shapes["v"][0]))])
            self.qkv_bias = torch.from_numpy(full).to(dev)
        else:
            self.qkv_bias = None
        self.o_bias = None if o_bias is None else torch.from_numpy(np.asarray(o_bias, np.float32)).to(dev)

    @staticmethod
    def random(model, rotation_matrix, seed: int = 0, scale: float | None = None, ctx=None) -> "Weights":
        """weights.py:112-133: N(0, 1) float32 times 1/sqrt(hidden) (float64), in q, k, v, o order."""
        rng = np.random.default_rng(seed)
        s = scale if scale is not None else 1.0 / np.sqrt(model.hidden_size)

        def w(shape):
            return rng.standard_normal(shape).astype(np.float32) * s
        return Weights(w((model.q_out_features, model.hidden_size)),
                       w((model.kv_out_features, model.hidden_size)),
                       w((model.kv_out_features, model.hidden_size)),
                       w((model.hidden_size, model.q_out_features)), model, rotation_matrix, ctx=ctx)


class HostHalf:
    """The per-token host work of kernel.py:198-249 and :348-356, on the GPU."""

    def __init__(self, model, weights: Weights, *, cast_after_rope: bool = True, ctx=None) -> None:
        import torch
        self.model = model
        self.weights = weights
        self.ctx = ctx or weights.ctx
        self.cast_after_rope = cast_after_rope
        self.rope = RoPE.build(model.head_dim, model.max_position, model.rope_theta, ROPE_FRAC,
                               model.rope_scaling)
        dev = self.ctx.torch_device
        self._cos = torch.from_numpy(self.rope.cos).to(dev)
        self._sin = torch.from_numpy(self.rope.sin).to(dev)
        self.attn_scale = 1.0 / np.sqrt(model.head_dim)           # kernel.py:103
        self.last_saturated = 0

    def project_qkv(self, x):
        """(n, hidden) float32 -> (n, (Hq + 2 Hkv) d) float32, ops/project.py:21-52."""
        import torch
        m = self.model
        x = self.ctx.to_device(x, torch.float32).reshape(-1, m.hidden_size).contiguous()
        n = x.shape[0]
        width = m.q_out_features + 2 * m.kv_out_features
        p = torch.empty((n, width), dtype=torch.float32, device=self.ctx.torch_device)
        _lib.check(self.ctx.lib.insitu_project(self.ctx.handle, ptr(self.weights.qkv), width, m.hidden_size,
                                               ptr(x), n, None, ptr(p)))
        self._keep = x
        return p

    def wire(self, x, positions, *, counts: bool = True):
        """kernel.py:198-249: hidden states (n, hidden) to the Q8.16 wire rows
        q (n, Hq, d), k and v (n, Hkv, d), int32 torch tensors on the device."""
        import torch
        m = self.model
        x = self.ctx.to_device(x, torch.float32).reshape(-1, m.hidden_size).contiguous()
        n = int(x.shape[0])
        positions = np.asarray(positions, dtype=np.int64).reshape(n)
        if n and (positions.min() < 0 or positions.max() >= m.max_position):
            # rope.py:163-167; checked here so that counts=False needs no read-back
            raise _lib.FormatError(_lib.ERANGE, f"position {int(positions.max())} beyond the RoPE "
                                   f"table (max_position {m.max_position})")
        # consecutive positions (a decode step, a prompt) go as their first value
        consecutive = n == 0 or bool(np.all(np.diff(positions) == 1))
        pos = None if consecutive else self.ctx.to_device(positions, torch.int64)
        pos0 = int(positions[0]) if n else 0
        dev = self.ctx.torch_device
        q = torch.empty((n, m.num_heads, m.head_dim), dtype=torch.int32, device=dev)
        k = torch.empty((n, m.num_kv_heads, m.head_dim), dtype=torch.int32, device=dev)
        v = torch.empty_like(k)
        cnt = (ctypes.c_uint64 * 2)() if counts else None
        bias = self.weights.qkv_bias
        width = m.q_out_features + 2 * m.kv_out_features
        p = torch.empty((n, width), dtype=torch.float32, device=dev)
        # the projection and the seam in one launch for a decode step (kernel.py:198-249)
        _lib.check(self.ctx.lib.insitu_project_seam(
            self.ctx.handle, ptr(self.weights.qkv), m.hidden_size, ptr(x), n,
            ptr(bias) if bias is not None else None, m.num_heads, m.num_kv_heads, m.head_dim,
            ptr(pos) if pos is not None else None, pos0, ptr(self._cos), ptr(self._sin),
            m.max_position, ROPE_FRAC, self.attn_scale, 1 if self.cast_after_rope else 0, ptr(p),
            ptr(q), ptr(k), ptr(v), cnt))
        if cnt is not None:
            self.last_saturated = int(cnt[0])
        self._keep = (x, p, pos)
        return q, k, v

    def output(self, out):
        """kernel.py:348-356: the Q16 out rows (n, Hq * d) to (n, hidden) float32."""
        import torch
        m = self.model
        o = self.ctx.to_device(out, torch.int32).reshape(-1, m.q_out_features).contiguous()
        n = o.shape[0]
        y = torch.empty((n, m.hidden_size), dtype=torch.float32, device=self.ctx.torch_device)
        bias = self.weights.o_bias
        _lib.check(self.ctx.lib.insitu_output_projection(
            self.ctx.handle, ptr(o), n, m.q_out_features, 16, ptr(self.weights.o), m.hidden_size,
            ptr(bias) if bias is not None else None, ptr(y)))
        self._keep_o = o
        return y
