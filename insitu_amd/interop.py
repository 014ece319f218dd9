"""Cache images in and out of the device, and a byte diff of two caches.

DdrLayout mirrors hw/ddr_layout.py:97-274 of the reference on the host side:
the device's plane layout (insitu_cache_layout) as an address map, with
image() (rows -> plane image, :227-248), row_at() (:250-257) and describe()
(:261-274). With CompressedCache.image/load_image (insitu_read_image /
insitu_load_image, the CMD_LOAD of host/attn_proto.py:75-78) a cache written
by the reference's host can be installed on the GPU byte for byte, and a GPU
cache read back for the reference's tools.

cache_diff is experiments/cache_diff.py:91-126 without the board: compare
stored rows with the host's, byte for byte, and name the field (key codes,
value codes, norms) of every row that differs, which names the encode-or-write
path that wrote it.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

BEAT_BYTES = 16


@dataclass(frozen=True)
class DdrLayout:
    """One sequence region: heads consecutive, each head's planes consecutive,
    every plane the same span; token t of plane p at plane_base + t * width."""

    plane_width: tuple
    plane_span: int
    n_kv_heads: int
    capacity: int
    fields: tuple            # (lo, hi) row-byte ranges: key codes, value codes, norms
    base: int = 0

    @classmethod
    def for_cache(cls, cache) -> "DdrLayout":
        """The layout the device uses for `cache` (a CompressedCache)."""
        d = cache.layout()
        q = cache.quant
        kb = cache.head_dim * q.key_bits // 8
        vb = cache.head_dim * q.value_bits // 8
        return cls(tuple(d["plane_width"]), d["plane_span"][0], d["n_kv_heads"], d["capacity"],
                   ((0, kb), (kb, kb + vb), (kb + vb, d["row_bytes"])))

    @classmethod
    def from_describe(cls, d: dict, fields: tuple) -> "DdrLayout":
        """From describe()'s dictionary (the reference's ddr_map.json)."""
        spans = set(d["plane_span"])
        if len(spans) != 1:
            raise ValueError("planes of unequal span")
        return cls(tuple(d["plane_width"]), spans.pop(), d["n_kv_heads"], d["capacity"],
                   tuple(tuple(f) for f in fields), d.get("base", 0))

    @property
    def row_bytes(self) -> int:
        return sum(self.plane_width)

    @property
    def n_ports(self) -> int:
        return len(self.plane_width)

    @property
    def head_stride(self) -> int:
        return self.n_ports * self.plane_span

    @property
    def total_bytes(self) -> int:
        return self.n_kv_heads * self.head_stride

    def _lo(self) -> np.ndarray:
        return np.concatenate([[0], np.cumsum(self.plane_width)[:-1]]).astype(np.int64)

    def plane_base(self, head: int, p: int) -> int:
        return self.base + head * self.head_stride + p * self.plane_span

    def token_addr(self, head: int, p: int, token: int) -> int:
        return self.plane_base(head, p) + token * self.plane_width[p]

    def image(self, buf) -> np.ndarray:
        """(tokens, heads, row_bytes) rows -> the plane image (zeros past the tokens)."""
        buf = np.asarray(buf, dtype=np.uint8)
        n, heads, rb = buf.shape
        if rb != self.row_bytes:
            raise ValueError(f"row is {rb} B, layout is built for {self.row_bytes}")
        if n > self.capacity:
            raise ValueError(f"{n} tokens exceeds capacity {self.capacity}")
        if heads != self.n_kv_heads:
            raise ValueError(f"{heads} kv heads, layout has {self.n_kv_heads}")
        img = np.zeros(self.total_bytes, dtype=np.uint8)
        for h in range(heads):
            for p, (lo, w) in enumerate(zip(self._lo(), self.plane_width)):
                a = self.plane_base(h, p) - self.base
                img[a:a + n * w] = buf[:, h, lo:lo + w].reshape(-1)
        return img

    def row_at(self, img, head: int, token: int) -> np.ndarray:
        """Reassemble one row out of its planes."""
        img = np.asarray(img, dtype=np.uint8)
        return np.concatenate([img[self.token_addr(head, p, token) - self.base:][:w]
                               for p, w in enumerate(self.plane_width)])

    def rows(self, img, n: int) -> np.ndarray:
        """Every row of tokens 0 .. n-1: (n, heads, row_bytes), the inverse of image()."""
        img = np.asarray(img, dtype=np.uint8).reshape(-1)
        if img.size < self.total_bytes:
            raise ValueError(f"image holds {img.size} B, the layout spans {self.total_bytes}")
        if n > self.capacity:
            raise ValueError(f"{n} tokens exceeds capacity {self.capacity}")
        out = np.empty((n, self.n_kv_heads, self.row_bytes), dtype=np.uint8)
        for h in range(self.n_kv_heads):
            for p, (lo, w) in enumerate(zip(self._lo(), self.plane_width)):
                a = self.plane_base(h, p) - self.base
                out[:, h, lo:lo + w] = img[a:a + n * w].reshape(n, w)
        return out

    def describe(self) -> dict:
        return {
            "row_bytes": self.row_bytes, "beat_bytes": BEAT_BYTES, "n_ports": self.n_ports,
            "plane_width": list(self.plane_width), "plane_span": [self.plane_span] * self.n_ports,
            "head_stride": self.head_stride, "capacity": self.capacity,
            "n_kv_heads": self.n_kv_heads, "base": self.base, "total_bytes": self.total_bytes,
            "bytes_per_cycle": self.row_bytes,
        }


FIELD_NAMES = ("key", "value", "norms")


@dataclass
class RowDiff:
    head: int
    token: int
    fields: list
    n_bytes: int
    got: np.ndarray
    want: np.ndarray


@dataclass
class DiffReport:
    n_tokens: int
    n_kv_heads: int
    rows: list = field(default_factory=list)

    @property
    def match(self) -> bool:
        return not self.rows

    def verdict(self) -> str:
        """experiments/cache_diff.py:114-121: where to look next."""
        if self.match:
            return ("every stored row matches the host byte for byte: the caches agree, "
                    "so a divergence is in the scan, not in what was written")
        fields = sorted({f for r in self.rows for f in r.fields}, key=FIELD_NAMES.index)
        return (f"{len(self.rows)} of {self.n_tokens * self.n_kv_heads} stored rows differ, in "
                f"{'+'.join(fields)}: that field's encode-or-write path is wrong; the scan "
                f"reads exactly what was put there")


def cache_diff(got_rows, want_rows, fields) -> DiffReport:
    """Compare (tokens, heads, row_bytes) rows; name the differing fields per row."""
    got = np.asarray(got_rows, dtype=np.uint8)
    want = np.asarray(want_rows, dtype=np.uint8)
    if got.shape != want.shape:
        raise ValueError(f"row arrays differ in shape: {got.shape} vs {want.shape}")
    n, heads, _ = got.shape
    rep = DiffReport(n, heads)
    bad = np.argwhere((got != want).any(axis=-1))
    for t, h in sorted(bad.tolist(), key=lambda th: (th[1], th[0])):
        g, w = got[t, h], want[t, h]
        which = [nm for nm, (lo, hi) in zip(FIELD_NAMES, fields) if not np.array_equal(g[lo:hi], w[lo:hi])]
        rep.rows.append(RowDiff(h, t, which, int(np.count_nonzero(g != w)), g.copy(), w.copy()))
    return rep


def diff_device_cache(cache, want_rows, seq: int = 0) -> DiffReport:
    """Read the device's plane image of one sequence, reassemble its rows with
    row_at's address map, and diff them against the host's rows."""
    lay = DdrLayout.for_cache(cache)
    want = np.asarray(want_rows, dtype=np.uint8)
    got = lay.rows(cache.image(seq), want.shape[0])
    return cache_diff(got, want, lay.fields)
