"""Plane layout of the compressed cache (oracle; test infrastructure only).

Restates hw/ddr_layout.py:75-274: each row is split at its field boundaries
(key codes, value codes, norms) and then into <=16-byte planes; every plane of
a head gets the widest plane's span rounded up to 4 KB; heads are consecutive.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

BEAT_BYTES = 16
PAGE = 4096


@dataclass(frozen=True)
class DdrLayout:
    row_bytes: int
    n_kv_heads: int
    capacity: int
    base: int = 0
    fields: tuple = ()

    @classmethod
    def for_format(cls, fmt, n_kv_heads: int, capacity: int, base: int = 0):
        """ddr_layout.py:110-124."""
        kb, vb, nb = fmt.key_bytes, fmt.value_bytes, 2 * (fmt.norm_bits // 8)
        return cls(kb + vb + nb, n_kv_heads, capacity, base,
                   ((0, kb), (kb, kb + vb), (kb + vb, kb + vb + nb)))

    @property
    def planes(self):
        """ddr_layout.py:148-163: list of (lo, hi) row-byte ranges."""
        fields = self.fields or ((0, self.row_bytes),)
        out = []
        for lo, hi in fields:
            a = lo
            while a < hi:
                b = min(a + BEAT_BYTES, hi)
                out.append((a, b))
                a = b
        return out

    @property
    def span(self) -> int:
        """ddr_layout.py:169-196: equal span, widest plane's bytes rounded to a page."""
        raw = max(self.capacity * (hi - lo) for lo, hi in self.planes)
        return (raw + PAGE - 1) // PAGE * PAGE

    @property
    def head_stride(self) -> int:
        return len(self.planes) * self.span

    @property
    def total_bytes(self) -> int:
        return self.n_kv_heads * self.head_stride

    def plane_base(self, head: int, p: int) -> int:
        """ddr_layout.py:198-211."""
        return self.base + head * self.head_stride + p * self.span

    def token_addr(self, head: int, p: int, token: int) -> int:
        lo, hi = self.planes[p]
        return self.plane_base(head, p) + token * (hi - lo)

    def image(self, buf: np.ndarray) -> np.ndarray:
        """ddr_layout.py:227-248: (tokens, heads, row_bytes) rows -> plane image."""
        buf = np.asarray(buf, dtype=np.uint8)
        n, heads, rb = buf.shape
        if rb != self.row_bytes or n > self.capacity or heads != self.n_kv_heads:
            raise ValueError("rows do not match the layout")
        img = np.zeros(self.total_bytes, dtype=np.uint8)
        for h in range(heads):
            for p, (lo, hi) in enumerate(self.planes):
                start = self.plane_base(h, p) - self.base
                chunk = buf[:n, h, lo:hi].reshape(-1)
                img[start:start + chunk.size] = chunk
        return img

    def row_at(self, img, head: int, token: int) -> np.ndarray:
        """ddr_layout.py:250-257."""
        img = np.asarray(img, dtype=np.uint8)
        parts = []
        for p, (lo, hi) in enumerate(self.planes):
            a = self.token_addr(head, p, token) - self.base
            parts.append(img[a:a + hi - lo])
        return np.concatenate(parts)

    def describe(self) -> dict:
        """ddr_layout.py:261-274."""
        return {
            "row_bytes": self.row_bytes, "beat_bytes": BEAT_BYTES,
            "n_ports": len(self.planes),
            "plane_width": [hi - lo for lo, hi in self.planes],
            "plane_span": [self.span] * len(self.planes),
            "head_stride": self.head_stride, "capacity": self.capacity,
            "n_kv_heads": self.n_kv_heads, "base": self.base,
            "total_bytes": self.total_bytes, "bytes_per_cycle": self.row_bytes,
        }
