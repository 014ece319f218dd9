"""The KV cache interface and the HBM-resident compressed cache.

KVCache mirrors cache/base.py:29-81 of the reference; CompressedCache mirrors
cache/compressed.py:42-132, with the packed rows living in device memory in
the plane layout of hw/ddr_layout.py (fields split into <=16-byte planes,
equal 4 KB-aligned spans, head-major), one region per sequence.

`view`/`view_from_buffer`/`buf` read the device bytes back to the host and
decode them (tests, diffing); the attention path never does.
"""

from __future__ import annotations

import abc
import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from .codebook import Codebook
from .config import FixedFormat, QuantConfig
from .rotate import Rotation
from .runtime import default_context, i64p, ptr


class KVCache(abc.ABC):
    """cache/base.py:29-81: fixed capacity, causal-order views."""

    def __init__(self, n_kv_heads: int, head_dim: int, capacity: int) -> None:
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim
        self.capacity = capacity

    @property
    @abc.abstractmethod
    def bytes_per_token(self) -> int:
        """One token, all KV heads."""

    @abc.abstractmethod
    def append_wire(self, k_wire, v_wire, *, seq: int | None = None) -> None:
        """kernel.py:271-272 + :283-284 in one launch: rotate wire k/v rows with the
        cache's rotation and append them (as append_rotated after Rotation.apply).

        batch == 1 (or `seq` given): (tokens, n_kv_heads, d); otherwise (batch, tokens,
        n_kv_heads, d). Raises ValueError past capacity.
        """
        import torch
        k = self.ctx.to_device(k_wire, torch.int32)
        v = self.ctx.to_device(v_wire, torch.int32)
        if k.shape != v.shape:
            raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} differ")
        if seq is None and self.batch == 1 and k.dim() == 3:
            seq = 0
        if seq is not None:
            if k.dim() != 3 or k.shape[1:] != (self.n_kv_heads, self.head_dim):
                raise ValueError(f"expected (tokens, {self.n_kv_heads}, {self.head_dim}), "
                                 f"got {tuple(k.shape)}")
            n = int(k.shape[0])
        else:
            if k.dim() != 4 or k.shape[0] != self.batch or \
                    k.shape[2:] != (self.n_kv_heads, self.head_dim):
                raise ValueError(f"expected ({self.batch}, tokens, {self.n_kv_heads}, "
                                 f"{self.head_dim}), got {tuple(k.shape)}")
            n = int(k.shape[1])
        _lib.check(self.ctx.lib.insitu_append_wire(self.handle, -1 if seq is None else seq,
                                                   ptr(k), ptr(v), n))
        self._keep = (k, v)     # keep inputs alive until the stream has consumed them

    def append(self, k, v, positions, trace=None) -> None:
        """Store (tokens, n_kv_heads, head_dim) of post-RoPE K and V."""

    @abc.abstractmethod
    def view(self, kv_head: int, trace=None):
        """Everything stored for one KV head, in causal order."""

    def stats(self) -> dict:
        return {"tokens": self.length, "capacity": self.capacity,
                "bytes_per_token": self.bytes_per_token,
                "bytes_resident": self.length * self.bytes_per_token}


@dataclass
class CompressedKV:
    """ops/quantize.py:99-118: one KV head's codes and norms (host arrays)."""

    k_idx: np.ndarray
    k_norm: np.ndarray
    v_idx: np.ndarray
    v_norm: np.ndarray

    @property
    def n_tokens(self) -> int:
        return int(np.prod(self.k_idx.shape[:-1])) if self.k_idx.ndim > 1 else 1

    def select(self, sl) -> "CompressedKV":
        return CompressedKV(self.k_idx[sl], self.k_norm[sl], self.v_idx[sl], self.v_norm[sl])


class DeviceKV:
    """compressed.py:95-121's view of one KV head, left where it lies: rows
    [0, stop) of (sequence, KV head) in device memory.

    CompressedAttention attends it on the GPU (kernel.py:385-392 hands the
    reference's attention `cache.view(h).select(slice(0, ctx))`). It also reads
    as the reference's CompressedKV: k_idx / k_norm / v_idx / v_norm read the
    rows back and decode them, once, for host code that wants the arrays.
    """

    def __init__(self, cache: "CompressedCache", kv_head: int, seq: int = 0, stop: int | None = None):
        self.cache = cache
        self.kv_head = int(kv_head)
        self.seq = int(seq)
        self.stop = cache.lengths()[seq] if stop is None else int(stop)
        self._host: CompressedKV | None = None

    @property
    def n_tokens(self) -> int:
        return self.stop

    def __len__(self) -> int:
        return self.stop

    def select(self, sl):
        """A prefix (slice(0, n), the causal context of a token) stays on the device;
        any other selection is a host CompressedKV."""
        if isinstance(sl, slice) and sl.step in (None, 1) and sl.start in (None, 0):
            stop = range(self.stop)[sl].stop if sl.stop is not None else self.stop
            return DeviceKV(self.cache, self.kv_head, self.seq, max(0, min(stop, self.stop)))
        return self.host().select(sl)

    def host(self) -> CompressedKV:
        if self._host is None:
            q = self.cache.quant
            rows = self.cache.read_rows(self.kv_head, 0, self.stop, self.seq)
            self._host = unpack_rows(rows, self.cache.head_dim, q.key_bits, q.value_bits, q.norm_bits)
        return self._host

    @property
    def k_idx(self) -> np.ndarray:
        return self.host().k_idx

    @property
    def k_norm(self) -> np.ndarray:
        return self.host().k_norm

    @property
    def v_idx(self) -> np.ndarray:
        return self.host().v_idx

    @property
    def v_norm(self) -> np.ndarray:
        return self.host().v_norm


def unpack_rows(buf: np.ndarray, d: int, key_bits: int, value_bits: int,
                norm_bits: int = 16) -> CompressedKV:
    """quantize.py:254-296: row bytes -> codes (LSB-first bitstreams) and sign-extended norms."""
    buf = np.asarray(buf, dtype=np.uint8)
    kb, vb, nb = d * key_bits // 8, d * value_bits // 8, norm_bits // 8

    def codes(field, bits):
        flat = field.reshape(-1, field.shape[-1])
        bitv = np.unpackbits(flat, axis=1, bitorder="little")[:, :d * bits].reshape(-1, d, bits)
        weights = (1 << np.arange(bits, dtype=np.uint16)).astype(np.uint16)
        return (bitv.astype(np.uint16) * weights).sum(-1).astype(np.uint8).reshape(
            *field.shape[:-1], d)

    def word(field):
        v = sum(field[..., i].astype(np.int64) << (8 * i) for i in range(nb))
        sign = 1 << (norm_bits - 1)
        return (v ^ sign) - sign

    o = 0
    k_idx = codes(buf[..., o:o + kb], key_bits); o += kb
    v_idx = codes(buf[..., o:o + vb], value_bits); o += vb
    k_norm = word(buf[..., o:o + nb]); o += nb
    v_norm = word(buf[..., o:o + nb])
    return CompressedKV(k_idx, k_norm, v_idx, v_norm)


class CompressedCache(KVCache):
    """cache/compressed.py:42-132 on the GPU, for `batch` sequences.

    `n_q_heads` is the query-head count the attention will serve (it fixes the
    GQA group size); it defaults to `n_kv_heads * 4`, the Llama-3 ratio.
    """

    def __init__(self, n_kv_heads: int, head_dim: int, capacity: int,
                 quant: QuantConfig, fmt: FixedFormat | None = None, qk_frac: int | None = None,
                 *, batch: int = 1, n_q_heads: int | None = None, chunk_tokens: int = 0,
                 ctx=None) -> None:
        super().__init__(n_kv_heads, head_dim, capacity)
        # tokens per chunk of the chunked attend: 0 (the default, 1,024) or 512, which doubles
        # the workgroups that walk a flat softmax's candidates
        self.chunk_tokens = chunk_tokens
        self.ctx = ctx or default_context()
        self.quant = quant
        self.fmt = fmt or FixedFormat()
        self.batch = batch
        self.n_q_heads = n_q_heads if n_q_heads is not None else n_kv_heads * 4
        self.rotation = Rotation.for_quant(quant, head_dim)
        self.key_codebook = Codebook.build(quant.codebook, quant.key_bits,
                                           self.fmt.centroid_frac, quant.symmetric)
        self.value_codebook = Codebook.build(quant.codebook, quant.value_bits,
                                             self.fmt.centroid_frac, quant.symmetric)
        self._row = quant.bytes_per_token(head_dim)
        if self.fmt.centroid_frac + quant.norm_frac < self.fmt.qk_frac:
            raise ValueError("centroid_frac + norm_frac is below qk_frac; the threshold "
                             "comparison would have to truncate x (quantize.py:150-156)")
        self.format = self._format()
        kc = np.ascontiguousarray(self.key_codebook.centroids, dtype=np.int64)
        kbd = np.ascontiguousarray(self.key_codebook.boundaries, dtype=np.int64)
        vc = np.ascontiguousarray(self.value_codebook.centroids, dtype=np.int64)
        vbd = np.ascontiguousarray(self.value_codebook.boundaries, dtype=np.int64)
        desc = _lib.CacheDesc()
        desc.capacity = capacity
        desc.batch = batch
        desc.n_kv_heads = n_kv_heads
        desc.n_q_heads = self.n_q_heads
        desc.chunk_tokens = chunk_tokens
        desc.fmt = self.format
        desc.key_centroids_host = i64p(kc)
        desc.key_bounds_host = i64p(kbd)
        desc.value_centroids_host = i64p(vc)
        desc.value_bounds_host = i64p(vbd)
        h = ctypes.c_void_p()
        _lib.check(self.ctx.lib.insitu_cache_create(self.ctx.handle, ctypes.byref(desc),
                                                    ctypes.byref(h)))
        self.handle = h
        lay = _lib.Layout()
        _lib.check(self.ctx.lib.insitu_cache_layout(self.handle, ctypes.byref(lay)))
        self._layout = lay

    def _format(self) -> "_lib.Format":
        f = _lib.Format()
        f.head_dim = self.head_dim
        f.key_bits = self.quant.key_bits
        f.value_bits = self.quant.value_bits
        f.norm_bits = self.quant.norm_bits
        f.norm_frac = self.quant.norm_frac
        f.qk_frac = self.fmt.qk_frac
        f.qk_width = self.fmt.qk_width
        f.centroid_frac = self.fmt.centroid_frac
        f.acc_frac = self.fmt.acc_frac
        f.acc_width = self.fmt.acc_width
        f.score_width = self.fmt.score_width
        f.prob_frac = self.fmt.prob_frac
        f.exp_lut_bits = self.fmt.exp_lut_bits
        self.rotation.fill_format(f)
        return f

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.ctx.lib.insitu_cache_destroy(self.handle)
            self.handle = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    # -- the KVCache interface ------------------------------------------------

    @property
    def row_bytes(self) -> int:
        return self._row

    @property
    def bytes_per_token(self) -> int:
        return self._row * self.n_kv_heads

    def lengths(self) -> list[int]:
        out = []
        for b in range(self.batch):
            v = ctypes.c_int64()
            _lib.check(self.ctx.lib.insitu_cache_length(self.handle, b, ctypes.byref(v)))
            out.append(int(v.value))
        return out

    @property
    def length(self) -> int:
        """Sequence 0's length (the reference cache holds one sequence)."""
        return self.lengths()[0]

    def append_rotated(self, k_rot, v_rot, trace=None, *, seq: int | None = None) -> None:
        """compressed.py:64-86: encode, pack and write rows at `length`.

        batch == 1 (or `seq` given): k_rot/v_rot are (tokens, n_kv_heads, d);
        otherwise (batch, tokens, n_kv_heads, d). Raises ValueError past capacity.
        """
        import torch
        k = self.ctx.to_device(k_rot, torch.int32)
        v = self.ctx.to_device(v_rot, torch.int32)
        if k.shape != v.shape:
            raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} differ")
        if seq is None and self.batch == 1 and k.dim() == 3:
            seq = 0
        if seq is not None:
            if k.dim() != 3 or k.shape[1:] != (self.n_kv_heads, self.head_dim):
                raise ValueError(f"expected (tokens, {self.n_kv_heads}, {self.head_dim}), "
                                 f"got {tuple(k.shape)}")
            _lib.check(self.ctx.lib.insitu_append_seq(self.handle, seq, ptr(k), ptr(v),
                                                      int(k.shape[0])))
        else:
            if k.dim() != 4 or k.shape[0] != self.batch or \
                    k.shape[2:] != (self.n_kv_heads, self.head_dim):
                raise ValueError(f"expected ({self.batch}, tokens, {self.n_kv_heads}, "
                                 f"{self.head_dim}), got {tuple(k.shape)}")
            _lib.check(self.ctx.lib.insitu_append(self.handle, ptr(k), ptr(v), int(k.shape[1])))
        self._keep = (k, v)     # keep inputs alive until the stream has consumed them

    def append_wire(self, k_wire, v_wire, *, seq: int | None = None) -> None:
        """kernel.py:271-272 + :283-284 in one launch: rotate wire k/v rows with the
        cache's rotation and append them (as append_rotated after Rotation.apply).

        batch == 1 (or `seq` given): (tokens, n_kv_heads, d); otherwise (batch, tokens,
        n_kv_heads, d). Raises ValueError past capacity.
        """
        import torch
        k = self.ctx.to_device(k_wire, torch.int32)
        v = self.ctx.to_device(v_wire, torch.int32)
        if k.shape != v.shape:
            raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} differ")
        if seq is None and self.batch == 1 and k.dim() == 3:
            seq = 0
        if seq is not None:
            if k.dim() != 3 or k.shape[1:] != (self.n_kv_heads, self.head_dim):
                raise ValueError(f"expected (tokens, {self.n_kv_heads}, {self.head_dim}), "
                                 f"got {tuple(k.shape)}")
            n = int(k.shape[0])
        else:
            if k.dim() != 4 or k.shape[0] != self.batch or \
                    k.shape[2:] != (self.n_kv_heads, self.head_dim):
                raise ValueError(f"expected ({self.batch}, tokens, {self.n_kv_heads}, "
                                 f"{self.head_dim}), got {tuple(k.shape)}")
            n = int(k.shape[1])
        _lib.check(self.ctx.lib.insitu_append_wire(self.handle, -1 if seq is None else seq,
                                                   ptr(k), ptr(v), n))
        self._keep = (k, v)     # keep inputs alive until the stream has consumed them

    def append(self, k, v, positions, trace=None) -> None:
        raise NotImplementedError(
            "CompressedCache stores rotated tokens; call append_rotated. Rotating inside "
            "the cache would mean the dense baseline and the compressed path rotate in two "
            "different places.")

    def read_rows(self, kv_head: int, t0: int = 0, n: int | None = None, seq: int = 0) -> np.ndarray:
        """The packed rows as the device holds them: uint8 (n, row_bytes)."""
        if n is None:
            n = self.lengths()[seq] - t0
        out = np.zeros((n, self._row), dtype=np.uint8)
        _lib.check(self.ctx.lib.insitu_read_rows(self.handle, seq, kv_head, t0, n,
                                                 out.ctypes.data_as(ctypes.c_void_p)))
        return out

    def load_rows(self, rows: np.ndarray, kv_head: int, t0: int = 0, seq: int = 0) -> None:
        """Write packed rows verbatim (CMD_LOAD, attn_proto.py:75-78). Lengths are unchanged."""
        rows = np.ascontiguousarray(rows, dtype=np.uint8)
        if rows.ndim != 2 or rows.shape[1] != self._row:
            raise ValueError(f"rows must be (n, {self._row})")
        _lib.check(self.ctx.lib.insitu_load_rows(self.handle, seq, kv_head, t0, rows.shape[0],
                                                 rows.ctypes.data_as(ctypes.c_void_p)))

    def image(self, seq: int = 0) -> np.ndarray:
        """The raw plane image of one sequence (DdrLayout.image, ddr_layout.py:227-248)."""
        out = np.zeros(self._layout.seq_stride, dtype=np.uint8)
        _lib.check(self.ctx.lib.insitu_read_image(self.handle, seq,
                                                  out.ctypes.data_as(ctypes.c_void_p), out.size))
        return out

    def load_image(self, img: np.ndarray, seq: int = 0) -> None:
        """Install a plane image verbatim (CMD_LOAD); lengths are unchanged."""
        img = np.ascontiguousarray(img, dtype=np.uint8).reshape(-1)
        _lib.check(self.ctx.lib.insitu_load_image(self.handle, seq,
                                                  img.ctypes.data_as(ctypes.c_void_p), img.size))

    def set_length(self, n: int, seq: int = 0) -> None:
        _lib.check(self.ctx.lib.insitu_cache_set_length(self.handle, seq, n))

    def pin_kernel(self, path: str) -> None:
        """Test hook: the kernel of sequential-mode attends on this cache, "auto" (the
        decode step's own kernel for insitu_step where it handles the format, the chunked
        attend where it handles the format and capacity, the scan attend elsewhere),
        "scan", "chunked" (the decode step too) or "step" (the decode step's own kernel).
        Raises if that kernel does not handle the cache."""
        code = {"auto": _lib.PATH_AUTO, "scan": _lib.PATH_SCAN, "chunked": _lib.PATH_CHUNKED,
                "step": _lib.PATH_STEP}[path]
        _lib.check(self.ctx.lib.insitu_cache_debug(self.handle, _lib.DEBUG_PATH, code))

    @property
    def buf(self) -> np.ndarray:
        """(length, n_kv_heads, row_bytes) of sequence 0, read from the device."""
        n = self.length
        out = np.zeros((n, self.n_kv_heads, self._row), dtype=np.uint8)
        for h in range(self.n_kv_heads):
            out[:, h] = self.read_rows(h, 0, n)
        return out

    def view(self, kv_head: int, trace=None, n_reads: int = 1, seq: int = 0) -> DeviceKV:
        """compressed.py:95-121: one KV head in causal order, as a device view
        (DeviceKV). trace and n_reads are the reference's cycle-model bookkeeping;
        the device records nothing into them."""
        if not 0 <= kv_head < self.n_kv_heads:
            raise IndexError(f"KV head {kv_head} of {self.n_kv_heads}")
        return DeviceKV(self, kv_head, seq)

    def view_from_buffer(self, kv_head: int, seq: int = 0) -> CompressedKV:
        rows = self.read_rows(kv_head, 0, None, seq)
        return unpack_rows(rows, self.head_dim, self.quant.key_bits, self.quant.value_bits,
                           self.quant.norm_bits)

    def reset(self) -> None:
        _lib.check(self.ctx.lib.insitu_cache_reset(self.handle))

    def layout(self) -> dict:
        """hw/ddr_layout.py:261-274 describe(), per sequence region."""
        lay = self._layout
        n = lay.n_planes
        return {
            "row_bytes": lay.row_bytes, "beat_bytes": 16, "n_ports": n,
            "plane_width": [lay.plane_width[i] for i in range(n)],
            "plane_span": [lay.plane_span] * n, "head_stride": lay.head_stride,
            "capacity": self.capacity, "n_kv_heads": self.n_kv_heads, "base": 0,
            "total_bytes": lay.seq_stride, "bytes_per_cycle": lay.row_bytes,
            "seq_stride": lay.seq_stride, "device_total_bytes": lay.total_bytes,
        }
