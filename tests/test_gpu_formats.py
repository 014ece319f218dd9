"""GPU: formats outside the d = 64 4b/2b decode step and its group of 4 query heads.

The reference attends any number of query heads per KV head (kernel.py:337-345) and any
key/value width (config.py:179-181); its default QuantConfig has 3-bit keys (config.py:141)
and its headline TinyLlama 8 query heads a KV head (config.py:122-125). Here:
  - 8 query heads a KV head in a format the scan attend does not take (3-bit keys) runs on
    the chunked attend, which sees each KV head as two chains of 4 query heads over the same
    rows (Geom.kv_shift);
  - 1 or 2 query heads a KV head run on the chunked attend with the chain's 4 query slots
    computing head h % G (Geom.gq): the duplicate slots' outputs and statistics are dropped,
    so the statistics must equal the oracle's for the real heads alone;
Every output is compared with oracle/c's attend_online over the same rows (and the decode
step's with the step loop's), bit for bit, with the statistics, and no head may fall back
to the serial path.
"""

import numpy as np
import pytest

from oracle import native
from oracle.quantize import Cache, Format
from oracle.rotate import rotate, signs_from_seed

pytestmark = pytest.mark.gpu


def _kv(rng, T, d=64, n_kv=8, scale=1 << 20):
    return (rng.integers(-scale, scale, size=(T, n_kv, d)),
            rng.integers(-scale, scale, size=(T, n_kv, d)))


def _want(k, v, q, f, G):
    n_kv = k.shape[1]
    host = Cache(n_kv, max(k.shape[0], 1), f)
    host.append_rotated(k, v)
    outs, sts = [], []
    for h in range(n_kv):
        o, s = native.attend_online(q[G * h:G * h + G], host.view(h), f)
        outs.append(o)
        sts.append(s)
    return np.concatenate(outs), sts


def _check(out, st, want, sts):
    np.testing.assert_array_equal(out, want)
    assert st.rescale_events == sum(s.rescale_events for s in sts)
    assert st.max_abs_acc == max(s.max_abs_acc for s in sts)
    assert st.max_abs_score == max(s.max_abs_score for s in sts)
    assert st.acc_overflows == sum(s.acc_overflows for s in sts)
    assert st.serial_fallbacks == 0


def _cache(ctx, capacity, *, d=64, kb=3, vb=2, n_kv=8, n_q=64, batch=1):
    from insitu_amd import QuantConfig
    from insitu_amd.cache import CompressedCache
    return CompressedCache(n_kv, d, capacity, QuantConfig(key_bits=kb, value_bits=vb), batch=batch,
                           n_q_heads=n_q, ctx=ctx)


@pytest.mark.parametrize("T", [1, 700, 1025, 9000])
@pytest.mark.parametrize("kb,vb", [(3, 2), (2, 3)])
def test_eight_query_heads_on_the_chunked_attend(ctx, T, kb, vb):
    from insitu_amd.attention import CompressedAttention
    f = Format(key_bits=kb, value_bits=vb)
    rng = np.random.default_rng(300 + T + kb)
    k, v = _kv(rng, T)
    c = _cache(ctx, T + 3, kb=kb, vb=vb)
    c.pin_kernel("chunked")                   # raises unless the chunked attend takes the cache
    c.pin_kernel("auto")
    c.append_rotated(k, v)
    q = rng.integers(-(1 << 22), 1 << 22, size=(64, 64))
    for mode in ("online", "split"):
        out, st = CompressedAttention(c).attend(q[None], mode)
        want, sts = _want(k, v, q, f, 8)
        _check(out.cpu().numpy()[0], st, want, sts)


def test_eight_query_heads_decode_steps_and_prefill(ctx):
    """insitu_step (two launches: the write kernel, then the attend) and the causal prefill
    on a 3b/2b cache with 8 query heads a KV head, against the oracle's step loop."""
    import torch
    from insitu_amd import _lib
    from insitu_amd.attention import CompressedAttention
    from insitu_amd.runtime import ptr
    f = Format(key_bits=3, value_bits=2)
    rng = np.random.default_rng(41)
    d, n_kv, n_q, T0, steps = 64, 4, 32, 1500, 3
    sg = signs_from_seed(d, 0, 1)
    kw = rng.integers(-(1 << 22), 1 << 22, size=(T0 + steps, n_kv, d))
    vw = rng.integers(-(1 << 22), 1 << 22, size=(T0 + steps, n_kv, d))
    qw = rng.integers(-(1 << 22), 1 << 22, size=(T0 + steps, n_q, d))
    kr = rotate(kw.reshape(-1, d), sg).reshape(kw.shape)
    vr = rotate(vw.reshape(-1, d), sg).reshape(vw.shape)
    qr = rotate(qw.reshape(-1, d), sg).reshape(qw.shape)
    c = _cache(ctx, T0 + steps, n_kv=n_kv, n_q=n_q)
    c.append_rotated(kr[:T0], vr[:T0])
    # the prefill: queries T0 - 3 .. T0 - 1 over rows 0 .. their own
    out, st = CompressedAttention(c).attend_prefill(ctx.to_device(qr[T0 - 3:T0], torch.int32), T0 - 3, "online")
    host = Cache(n_kv, T0 + steps, f)
    host.append_rotated(kr[:T0], vr[:T0])
    want = native.decode_steps(qr[T0 - 3:T0], [host.view(h) for h in range(n_kv)], f, base=T0 - 3)
    np.testing.assert_array_equal(out.cpu().numpy().reshape(want.shape), want)
    assert st.serial_fallbacks == 0
    # decode steps from the wire
    for i in range(steps):
        t = T0 + i
        o = torch.empty((1, n_q, d), dtype=torch.int32, device=ctx.torch_device)
        qd = ctx.to_device(qw[t][None], torch.int32)
        kd = ctx.to_device(kw[t][None], torch.int32)
        vd = ctx.to_device(vw[t][None], torch.int32)
        s = _lib.Stats()
        _lib.check(ctx.lib.insitu_step(c.handle, ptr(qd), ptr(kd), ptr(vd), ptr(o), 0, s))
        host.append_rotated(kr[t:t + 1], vr[t:t + 1])
        want = np.concatenate([native.attend_online(qr[t][8 * h:8 * h + 8], host.view(h), f)[0]
                               for h in range(n_kv)])
        np.testing.assert_array_equal(o.cpu().numpy()[0], want)
        assert s.serial_fallbacks == 0


def _check_all(out, st, want, sts):
    _check(out, st, want, sts)
    assert st.score_overflows == sum(s.score_overflows for s in sts)


@pytest.mark.parametrize("G", [1, 2])
@pytest.mark.parametrize("T", [1, 700, 9000])
def test_fewer_than_four_query_heads(ctx, G, T):
    from insitu_amd.attention import CompressedAttention
    f = Format()
    rng = np.random.default_rng(500 + 10 * T + G)
    k, v = _kv(rng, T)
    c = _cache(ctx, T + 3, kb=4, vb=2, n_q=8 * G)
    c.pin_kernel("chunked")                   # raises unless the chunked attend takes the cache
    c.pin_kernel("auto")
    c.append_rotated(k, v)
    q = rng.integers(-(1 << 22), 1 << 22, size=(8 * G, 64))
    q[0] = 1 << 26                               # large scores: overflows to count
    for mode in ("online", "split"):
        out, st = CompressedAttention(c).attend(q[None], mode)
        want, sts = _want(k, v, q, f, G)
        _check_all(out.cpu().numpy()[0], st, want, sts)
    out, st = CompressedAttention(c).attend(q[None], "two_pass")
    host = Cache(8, max(T, 1), f)
    host.append_rotated(k, v)
    want = np.concatenate([native.attend_two_pass(q[G * h:G * h + G], host.view(h), f)[0] for h in range(8)])
    np.testing.assert_array_equal(out.cpu().numpy()[0], want)
    assert st.serial_fallbacks == 0


def test_two_query_heads_decode_steps(ctx):
    import torch
    from insitu_amd import _lib
    from insitu_amd.runtime import ptr
    f = Format()
    rng = np.random.default_rng(43)
    d, n_kv, G, T0, steps = 64, 8, 2, 2100, 3
    sg = signs_from_seed(d, 0, 1)
    kw = rng.integers(-(1 << 22), 1 << 22, size=(T0 + steps, n_kv, d))
    vw = rng.integers(-(1 << 22), 1 << 22, size=(T0 + steps, n_kv, d))
    qw = rng.integers(-(1 << 22), 1 << 22, size=(T0 + steps, n_kv * G, d))
    kr = rotate(kw.reshape(-1, d), sg).reshape(kw.shape)
    vr = rotate(vw.reshape(-1, d), sg).reshape(vw.shape)
    qr = rotate(qw.reshape(-1, d), sg).reshape(qw.shape)
    c = _cache(ctx, T0 + steps, kb=4, vb=2, n_q=n_kv * G)
    c.append_rotated(kr[:T0], vr[:T0])
    host = Cache(n_kv, T0 + steps, f)
    host.append_rotated(kr[:T0], vr[:T0])
    for i in range(steps):
        t = T0 + i
        o = torch.empty((1, n_kv * G, d), dtype=torch.int32, device=ctx.torch_device)
        qd = ctx.to_device(qw[t][None], torch.int32)
        kd = ctx.to_device(kw[t][None], torch.int32)
        vd = ctx.to_device(vw[t][None], torch.int32)
        s = _lib.Stats()
        _lib.check(ctx.lib.insitu_step(c.handle, ptr(qd), ptr(kd), ptr(vd), ptr(o), 0, s))
        host.append_rotated(kr[t:t + 1], vr[t:t + 1])
        res = [native.attend_online(qr[t][G * h:G * h + G], host.view(h), f) for h in range(n_kv)]
        np.testing.assert_array_equal(o.cpu().numpy()[0], np.concatenate([r[0] for r in res]))
        assert s.serial_fallbacks == 0
        assert s.rescale_events == sum(r[1].rescale_events for r in res)
