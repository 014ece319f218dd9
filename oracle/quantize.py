"""Norm, threshold encode and the packed row format (oracle; test infrastructure only).

Restates ops/quantize.py:42-296 and the format constants of config.py:132-254.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .codebook import gaussian
from .fixed import I64, Q, lshift, rshift


@dataclass(frozen=True)
class Format:
    """The format numbers of config.py QuantConfig/FixedFormat that the path uses."""

    d: int = 64
    key_bits: int = 4
    value_bits: int = 2
    norm_bits: int = 16
    norm_frac: int = 9
    qk_frac: int = 16
    qk_width: int = 24
    centroid_frac: int = 15
    acc_frac: int = 16
    acc_width: int = 32
    score_width: int = 48
    prob_frac: int = 15
    exp_lut_bits: int = 8
    seed: int = 0
    rot_rounds: int = 1

    @property
    def threshold_frac(self) -> int:            # quantize.py:86-89
        return self.centroid_frac + self.norm_frac

    @property
    def score_shift(self) -> int:               # config.py:249-250
        return self.qk_frac + self.centroid_frac + self.norm_frac - self.acc_frac

    @property
    def acc_shift(self) -> int:                 # config.py:252-254
        return self.centroid_frac + self.norm_frac + self.prob_frac - self.acc_frac

    @property
    def key_bytes(self) -> int:
        return _code_bytes(self.d, self.key_bits)

    @property
    def value_bytes(self) -> int:
        return _code_bytes(self.d, self.value_bits)

    @property
    def row_bytes(self) -> int:                 # quantize.py:158-160, config.py:192-207
        return self.key_bytes + self.value_bytes + 2 * (self.norm_bits // 8)

    def codebooks(self):
        """(key_centroids, key_bounds, value_centroids, value_bounds)."""
        kc, kb = gaussian(self.key_bits, self.centroid_frac)
        vc, vb = gaussian(self.value_bits, self.centroid_frac)
        return kc, kb, vc, vb


def _code_bytes(d: int, bits: int) -> int:
    if (d * bits) % 8:
        raise ValueError(f"{d}*{bits} bits is not whole bytes")
    return d * bits // 8


def isqrt(x) -> np.ndarray:
    """Exact integer square root; quantize.py:42-60 (float seed, then corrected)."""
    a = np.asarray(x, dtype=I64)
    if np.any(a < 0):
        raise ValueError("isqrt of a negative value")
    r = np.sqrt(a.astype(np.float64)).astype(I64)
    r = np.maximum(r - 1, 0)
    for _ in range(3):
        r = np.where((r + 1) * (r + 1) <= a, r + 1, r)
    if not np.all((r * r <= a) & ((r + 1) * (r + 1) > a)):
        raise AssertionError("isqrt correction failed")
    return r


def norm_wire(x_rot, fmt: Format) -> np.ndarray:
    """quantize.py:164-181: isqrt(sum(x^2) // d) in Q(qk_frac), then half-even into Q(norm)."""
    sq = (np.asarray(x_rot, dtype=I64) ** 2).sum(axis=-1)
    norm = isqrt(sq // I64(fmt.d))
    return Q(fmt.norm_bits, fmt.norm_frac).requantize(norm, fmt.qk_frac, "even")


def encode_plane(x_rot, boundaries, norm, fmt: Format) -> np.ndarray:
    """quantize.py:183-196: code = #{i : (x << (thr_frac - qk_frac)) > norm * b_i}."""
    thr = np.asarray(norm, dtype=I64)[..., None, None] * np.asarray(boundaries, dtype=I64)
    xs = lshift(np.asarray(x_rot, dtype=I64), fmt.threshold_frac - fmt.qk_frac)
    return (xs[..., None] > thr).sum(axis=-1).astype(np.uint8)


@dataclass
class CompressedKV:
    """quantize.py:99-118: codes and norms for (..., d)."""

    k_idx: np.ndarray
    k_norm: np.ndarray
    v_idx: np.ndarray
    v_norm: np.ndarray

    def select(self, sl) -> "CompressedKV":
        return CompressedKV(self.k_idx[sl], self.k_norm[sl], self.v_idx[sl], self.v_norm[sl])


def encode(k_rot, v_rot, fmt: Format) -> CompressedKV:
    """quantize.py:198-212."""
    kc, kb, vc, vb = fmt.codebooks()
    kn = norm_wire(k_rot, fmt)
    vn = norm_wire(v_rot, fmt)
    return CompressedKV(encode_plane(k_rot, kb, kn, fmt), kn,
                        encode_plane(v_rot, vb, vn, fmt), vn)


def decode_plane(idx, norm, centroids, fmt: Format) -> np.ndarray:
    """quantize.py:216-220 (tests only)."""
    c = np.asarray(centroids, dtype=I64)[np.asarray(idx, dtype=I64)]
    return rshift(c * np.asarray(norm, dtype=I64)[..., None], fmt.threshold_frac - fmt.qk_frac)


def pack_codes(idx, bits: int) -> np.ndarray:
    """quantize.py:271-275: LSB-first bitstream of `bits`-wide codes, little-endian bytes."""
    idx = np.asarray(idx, dtype=np.uint8)
    flat = idx.reshape(-1, idx.shape[-1])
    bit = np.unpackbits(flat[:, :, None], axis=2, bitorder="little")[:, :, :bits]
    out = np.packbits(bit.reshape(flat.shape[0], -1), axis=1, bitorder="little")
    return out.reshape(*idx.shape[:-1], -1)


def unpack_codes(buf, bits: int, d: int) -> np.ndarray:
    """quantize.py:278-283."""
    buf = np.asarray(buf, dtype=np.uint8)
    flat = buf.reshape(-1, buf.shape[-1])
    bit = np.unpackbits(flat, axis=1, bitorder="little")[:, :d * bits].reshape(-1, d, bits)
    pad = np.zeros((*bit.shape[:2], 8 - bits), dtype=np.uint8)
    packed = np.packbits(np.concatenate([bit, pad], axis=2), axis=2, bitorder="little")
    return packed[..., 0].reshape(*buf.shape[:-1], d)


def pack_word(x, bits: int) -> np.ndarray:
    """quantize.py:286-289: two's-complement little-endian bytes."""
    nb = bits // 8
    a = np.asarray(x, dtype=I64) & ((I64(1) << I64(bits)) - 1)
    return np.stack([(a >> I64(8 * i)) & 0xFF for i in range(nb)], axis=-1).astype(np.uint8)


def unpack_word(buf, bits: int) -> np.ndarray:
    """quantize.py:292-296: sign-extended."""
    nb = bits // 8
    v = sum(np.asarray(buf)[..., i].astype(I64) << I64(8 * i) for i in range(nb))
    sign = I64(1) << I64(bits - 1)
    return (v ^ sign) - sign


def pack(kv: CompressedKV, fmt: Format) -> np.ndarray:
    """quantize.py:237-252: k codes | v codes | k_norm | v_norm."""
    return np.concatenate([
        pack_codes(kv.k_idx, fmt.key_bits),
        pack_codes(kv.v_idx, fmt.value_bits),
        pack_word(kv.k_norm, fmt.norm_bits),
        pack_word(kv.v_norm, fmt.norm_bits),
    ], axis=-1)


def unpack(buf, fmt: Format) -> CompressedKV:
    """quantize.py:254-264."""
    buf = np.asarray(buf, dtype=np.uint8)
    if buf.shape[-1] != fmt.row_bytes:
        raise ValueError(f"expected {fmt.row_bytes} B per token, got {buf.shape[-1]}")
    nb = fmt.norm_bits // 8
    kb, vb = fmt.key_bytes, fmt.value_bytes
    o = 0
    k_idx = unpack_codes(buf[..., o:o + kb], fmt.key_bits, fmt.d); o += kb
    v_idx = unpack_codes(buf[..., o:o + vb], fmt.value_bits, fmt.d); o += vb
    k_norm = unpack_word(buf[..., o:o + nb], fmt.norm_bits); o += nb
    v_norm = unpack_word(buf[..., o:o + nb], fmt.norm_bits)
    return CompressedKV(k_idx, k_norm, v_idx, v_norm)


@dataclass
class Cache:
    """cache/compressed.py:42-132 + cache/base.py:29-81, host-only: packed rows + shadow."""

    n_kv_heads: int
    capacity: int
    fmt: Format
    length: int = 0
    buf: np.ndarray = field(init=False)

    def __post_init__(self) -> None:
        self.buf = np.zeros((self.capacity, self.n_kv_heads, self.fmt.row_bytes), dtype=np.uint8)

    def append_rotated(self, k_rot, v_rot) -> None:
        k_rot = np.asarray(k_rot)
        n = k_rot.shape[0]
        if self.length + n > self.capacity:          # base.py:67-73
            raise ValueError(f"cache holds {self.length} of {self.capacity} tokens; "
                             f"cannot append {n}")
        kv = encode(k_rot, v_rot, self.fmt)
        self.buf[self.length:self.length + n] = pack(kv, self.fmt)
        self.length += n

    def view(self, kv_head: int) -> CompressedKV:
        return unpack(self.buf[:self.length, kv_head], self.fmt)

    def reset(self) -> None:
        self.length = 0
