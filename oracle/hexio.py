"""Readers for the reference's `$readmemh` golden files (oracle; test infrastructure only).

Conventions of hw/vectors.py:72-121 and :379-814: each line is one record,
printed MSB-first, so lane 0 / byte 0 / token 0 sits rightmost; values are
two's complement masked to the lane width; sub-word lanes are packed LSB-first.
"""

from __future__ import annotations

import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT_DIR = os.path.join(os.path.dirname(HERE), "tests", "golden", "tb_vectors")


def path(name: str, root: str | None = None) -> str:
    return os.path.join(root or DEFAULT_DIR, name)


def lines(name: str, root: str | None = None) -> list[str]:
    with open(path(name, root)) as f:
        return [ln.strip() for ln in f if ln.strip()]


def manifest(root: str | None = None) -> dict:
    with open(path("manifest.json", root)) as f:
        return json.load(f)


def _sext(v: int, bits: int) -> int:
    sign = 1 << (bits - 1)
    return (v ^ sign) - sign


def lanes(name: str, bits: int, count: int | None = None, signed: bool = True,
          root: str | None = None) -> np.ndarray:
    """Each line -> `count` lanes of `bits` bits, lane 0 in the low bits."""
    rows = []
    mask = (1 << bits) - 1
    for ln in lines(name, root):
        v = int(ln, 16)
        n = count if count is not None else (len(ln) * 4) // bits
        row = []
        for i in range(n):
            x = (v >> (i * bits)) & mask
            row.append(_sext(x, bits) if signed else x)
        rows.append(row)
    return np.array(rows, dtype=object).astype(np.int64) if rows else np.zeros((0, 0), np.int64)


def scalars(name: str, bits: int, signed: bool = True, root: str | None = None) -> np.ndarray:
    """One value per line."""
    return lanes(name, bits, 1, signed, root)[:, 0]


def bytes_rows(name: str, root: str | None = None) -> np.ndarray:
    """Lines of hex bytes, byte 0 rightmost -> uint8 (lines, nbytes)."""
    out = []
    for ln in lines(name, root):
        b = bytes.fromhex(ln)[::-1]
        out.append(np.frombuffer(b, dtype=np.uint8))
    return np.stack(out)


def pack_lanes(values, bits: int) -> bytes:
    """hw/vectors.py:72-93: signed ints -> LSB-first packed little-endian bytes."""
    acc, n, out = 0, 0, bytearray()
    mask = (1 << bits) - 1
    for v in np.asarray(values).reshape(-1):
        acc |= (int(v) & mask) << n
        n += bits
        while n >= 8:
            out.append(acc & 0xFF)
            acc >>= 8
            n -= 8
    if n:
        out.append(acc & 0xFF)
    return bytes(out)


def unpack_lanes(buf: bytes, bits: int, count: int) -> np.ndarray:
    """hw/vectors.py:96-105."""
    acc = int.from_bytes(buf, "little")
    mask = (1 << bits) - 1
    return np.array([_sext((acc >> (i * bits)) & mask, bits) for i in range(count)],
                    dtype=np.int64)
