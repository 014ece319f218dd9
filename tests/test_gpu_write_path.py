"""GPU: the write path (append_kernel) against the oracle's encoder and packer.

append_rotated (compressed.py:64-86: the norm, the threshold codes, the packed row in the
plane layout) and append_wire (kernel.py:271-272 + :283-284: Rotation.apply of the wire
k/v, then append_rotated) run on one kernel whose waves pack rows in turn. Every cache
byte is compared with the oracle's encode + pack of the same rows (quantize.py:164-296),
for formats whose encoder bisects sorted boundaries (2^bits - 1 of them) and for the
widths at the ends (1 and 8 bits), over row counts that leave waves with one row and with
several, and across sequences of a batch.
"""

import numpy as np
import pytest

from oracle.quantize import Format, encode, pack
from oracle.rotate import rotate, signs_from_seed

pytestmark = pytest.mark.gpu


def _cache(ctx, capacity, *, d=64, kb=4, vb=2, batch=1, n_kv=8):
    from insitu_amd import QuantConfig
    from insitu_amd.cache import CompressedCache
    return CompressedCache(n_kv, d, capacity, QuantConfig(key_bits=kb, value_bits=vb), batch=batch,
                           n_q_heads=4 * n_kv, ctx=ctx)


def _rows(c, seq, n, n_kv=8):
    return np.stack([c.read_rows(h, 0, n, seq=seq) for h in range(n_kv)], axis=1)


@pytest.mark.parametrize("d,kb,vb", [(64, 4, 2), (64, 3, 2), (128, 3, 3), (64, 1, 8), (128, 5, 2)])
@pytest.mark.parametrize("n", [1, 37, 3001])
def test_append_wire_is_rotate_then_append(ctx, d, kb, vb, n):
    f = Format(d=d, key_bits=kb, value_bits=vb)
    rng = np.random.default_rng(1000 * kb + 10 * vb + n)
    kw = rng.integers(-(1 << 23), 1 << 23, size=(n, 8, d))
    vw = rng.integers(-(1 << 23), 1 << 23, size=(n, 8, d))
    kw[0, 1] = 0                                   # a zero vector: norm 0, all-equal codes
    sg = signs_from_seed(d, 0, 1)
    kr = rotate(kw.reshape(-1, d), sg).reshape(n, 8, d)
    vr = rotate(vw.reshape(-1, d), sg).reshape(n, 8, d)
    want = pack(encode(kr, vr, f), f)
    a = _cache(ctx, n + 8, d=d, kb=kb, vb=vb)
    a.append_wire(kw, vw)
    b = _cache(ctx, n + 8, d=d, kb=kb, vb=vb)
    b.append_rotated(kr, vr)
    assert a.length == b.length == n
    np.testing.assert_array_equal(_rows(a, 0, n), want)
    np.testing.assert_array_equal(_rows(b, 0, n), want)


def test_append_wire_every_sequence_of_a_batch(ctx):
    d, n, batch = 64, 700, 3
    f = Format(d=d)
    rng = np.random.default_rng(5)
    kw = rng.integers(-(1 << 22), 1 << 22, size=(batch, n, 8, d))
    vw = rng.integers(-(1 << 22), 1 << 22, size=(batch, n, 8, d))
    c = _cache(ctx, 2048, batch=batch)
    c.append_wire(kw[:, :300], vw[:, :300])                 # every sequence
    c.append_wire(kw[1, 300:], vw[1, 300:], seq=1)         # one sequence
    assert c.lengths() == [300, n, 300]
    sg = signs_from_seed(d, 0, 1)
    for b in range(batch):
        m = n if b == 1 else 300
        kr = rotate(kw[b, :m].reshape(-1, d), sg).reshape(m, 8, d)
        vr = rotate(vw[b, :m].reshape(-1, d), sg).reshape(m, 8, d)
        np.testing.assert_array_equal(_rows(c, b, m), pack(encode(kr, vr, f), f))

