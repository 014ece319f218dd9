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



# -- the lane = row kernel against the lane-per-channel one and the oracle -----------------
#
# At d = 64 with 4/2- and 2/2-bit codes the append runs on append_rows_kernel (a row per
# lane, fp64 arithmetic on integers where it is exact, int64 where it is not); the debug
# setting INSITU_DEBUG_APPEND = 1 pins the lane-per-channel append_kernel. Rows cover the
# paths the lane = row kernel takes: ordinary rows, zero rows, one-channel rows, rows whose
# sum of squares reaches 2^53 (the int64 norm), INT32_MIN/MAX entries, and wire rows whose
# rotation leaves int32 (range errors, wrapped to int32, recounted by the whole wave).


def _extreme_rows(rng, n, d=64, wire=True):
    k = rng.integers(-(1 << 23), 1 << 23, size=(n, 8, d))
    sg = signs_from_seed(d, 0, 1)[0]
    for t in range(0, n, 7):
        h = t % 8
        kind = (t // 7) % 6
        if kind == 0:
            k[t, h] = 0
        elif kind == 1:
            k[t, h] = 0
            k[t, h, t % d] = (1 << 31) - 1
        elif kind == 2:                       # sum of squares >= 2^53 (int64 norm)
            k[t, h] = rng.choice([-1, 1], size=d) * (1 << 27)
        elif kind == 3:
            k[t, h, :8] = -(1 << 31)
            k[t, h, 8:16] = (1 << 31) - 1
        elif kind == 4 and wire:              # the signs aligned: channel 0 leaves int32
            k[t, h] = sg * ((1 << 31) - 1)
        elif kind == 5 and wire:              # half aligned: several channels leave int32
            k[t, h] = sg * ((1 << 31) - 1)
            k[t, h, d // 2:] = -k[t, h, d // 2:] // 2
    return k


def _wrap32(x):
    return ((np.asarray(x, dtype=np.int64) + (1 << 31)) % (1 << 32)) - (1 << 31)


def _append_stats(c):
    from insitu_amd import _lib
    st = _lib.Stats()
    _lib.check(c.ctx.lib.insitu_cache_stats(c.handle, st))
    return st.range_errors, st.serial_fallbacks


@pytest.mark.parametrize("kb,vb", [(4, 2), (2, 2)])
@pytest.mark.parametrize("n", [1, 63, 64, 65, 1000])
def test_lane_row_append_equals_lane_channel(ctx, kb, vb, n):
    from insitu_amd import _lib
    f = Format(key_bits=kb, value_bits=vb)
    rng = np.random.default_rng(100 * kb + n)
    kw, vw = _extreme_rows(rng, n), _extreme_rows(rng, n)[::-1].copy()
    caches = []
    for pin in (0, 1):
        c = _cache(ctx, n + 8, kb=kb, vb=vb)
        _lib.check(ctx.lib.insitu_cache_debug(c.handle, _lib.DEBUG_APPEND, pin))
        _append_stats(c)                                     # cleared
        c.append_wire(kw, vw)
        caches.append((c, _append_stats(c)))
    (a, sa), (b, sb) = caches
    np.testing.assert_array_equal(_rows(a, 0, n), _rows(b, 0, n))
    assert sa == sb
    # the oracle: rotate, wrap to int32 (counting what left it), encode and pack
    sg = signs_from_seed(64, 0, 1)
    kr = rotate(kw.reshape(-1, 64), sg).reshape(n, 8, 64)
    vr = rotate(vw.reshape(-1, 64), sg).reshape(n, 8, 64)
    outside = int(np.sum(kr != _wrap32(kr)) + np.sum(vr != _wrap32(vr)))
    assert sa == (outside, 0)
    if n >= 64:
        assert outside > 0
    # rows whose wrapped values' squares sum past int64 are left to the comparison above
    # (both kernels wrap alike; the oracle's isqrt refuses the wrapped negative sum)
    kw32, vw32 = _wrap32(kr), _wrap32(vr)
    sq = lambda x: (x.astype(np.float64) ** 2).sum(-1)
    ok = (sq(kw32) < 2.0 ** 62) & (sq(vw32) < 2.0 ** 62)
    assert ok.sum() >= 0.9 * ok.size
    want = pack(encode(np.where(ok[..., None], kw32, 0), np.where(ok[..., None], vw32, 0), f), f)
    np.testing.assert_array_equal(_rows(a, 0, n)[ok], want[ok])


@pytest.mark.parametrize("n", [1, 65, 700])
def test_lane_row_append_rotated_rows_against_the_oracle(ctx, n):
    # rotated rows in (insitu_append): the int64 norm where sum(x^2) >= 2^53, INT32_MIN/MAX
    f = Format()
    rng = np.random.default_rng(7 + n)
    k, v = _extreme_rows(rng, n, wire=False), _extreme_rows(rng, n, wire=False)[::-1].copy()
    c = _cache(ctx, n + 8)
    c.append_rotated(k, v)
    np.testing.assert_array_equal(_rows(c, 0, n), pack(encode(k, v, f), f))
    assert _append_stats(c) == (0, 0)


def test_lane_row_append_batch_and_offsets(ctx):
    # a batch of 3, every sequence then one, from different lengths: the lanes' (sequence,
    # token, KV head) and positions; tiles that cross sequences
    d, batch = 64, 3
    f = Format(d=d)
    rng = np.random.default_rng(11)
    kw = rng.integers(-(1 << 22), 1 << 22, size=(batch, 900, 8, d))
    vw = rng.integers(-(1 << 22), 1 << 22, size=(batch, 900, 8, d))
    c = _cache(ctx, 2048, batch=batch)
    c.append_wire(kw[:, :37], vw[:, :37])
    c.append_wire(kw[2, 37:900], vw[2, 37:900], seq=2)
    c.append_wire(kw[:, 37:101], vw[:, 37:101])
    assert c.lengths() == [101, 101, 964]
    sg = signs_from_seed(d, 0, 1)
    for b in range(batch):
        seqk = kw[b, :101] if b < 2 else np.concatenate([kw[2, :37], kw[2, 37:900], kw[2, 37:101]])
        seqv = vw[b, :101] if b < 2 else np.concatenate([vw[2, :37], vw[2, 37:900], vw[2, 37:101]])
        m = seqk.shape[0]
        kr = rotate(seqk.reshape(-1, d), sg).reshape(m, 8, d)
        vr = rotate(seqv.reshape(-1, d), sg).reshape(m, 8, d)
        np.testing.assert_array_equal(_rows(c, b, m), pack(encode(kr, vr, f), f))


@pytest.mark.parametrize("rounds", [1, 2])
@pytest.mark.parametrize("n", [1, 63, 64, 65, 777])
def test_lane_row_rotation_against_the_oracle(ctx, rounds, n):
    # insitu_rotate at d = 64 runs rotate_rows_kernel (a row per lane, fp64 FWHT): every
    # vector against the oracle's rotation wrapped to int32, on ordinary and extreme rows
    # (values leaving int32, INT32_MIN/MAX entries, zero and one-channel rows)
    from insitu_amd.rotate import Rotation
    rng = np.random.default_rng(31 * rounds + n)
    x = _extreme_rows(rng, n).reshape(-1, 64)[: max(n, 1)]
    rot = Rotation.from_seed(64, 0, rounds)
    want = _wrap32(rotate(x, signs_from_seed(64, 0, rounds)))
    np.testing.assert_array_equal(rot.apply(x, ctx).cpu().numpy(), want)
