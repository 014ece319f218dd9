"""GPU: the scan attend (attend_scan.hip) against the oracle.

The scan attend is the sequential-mode kernel for the caches the chunked attend
does not take: 8 query heads per KV head, and contexts past 512 chunks. A test
hook (CompressedCache.pin_kernel) also pins it on the chunked attend's formats,
so both kernels are checked on the same cases. Every output is compared with
oracle/c's attend_online over the same rows, bit for bit, and the statistics
with the oracle's.
"""

import numpy as np
import pytest

from oracle import native
from oracle.quantize import Cache, Format
from oracle.rotate import rotate, signs_from_seed

pytestmark = pytest.mark.gpu


def _cache(ctx, capacity, *, d=64, kb=4, vb=2, batch=1, n_kv=8, n_q=32, pin="scan"):
    from insitu_amd import QuantConfig
    from insitu_amd.cache import CompressedCache
    c = CompressedCache(n_kv, d, capacity, QuantConfig(key_bits=kb, value_bits=vb),
                        batch=batch, n_q_heads=n_q, ctx=ctx)
    c.pin_kernel(pin)
    return c


def _kv(rng, T, d=64, n_kv=8, scale=1 << 20):
    return (rng.integers(-scale, scale, size=(T, n_kv, d)),
            rng.integers(-scale, scale, size=(T, n_kv, d)))


def _want(k, v, q, f, G=4):
    """The oracle's attend_online per KV group (G query heads each), and its stats."""
    n_kv = k.shape[1]
    host = Cache(n_kv, max(k.shape[0], 1), f)
    host.append_rotated(k, v)
    outs, sts = [], []
    for h in range(n_kv):
        o, s = native.attend_online(q[G * h:G * h + G], host.view(h), f)
        outs.append(o)
        sts.append(s)
    return np.concatenate(outs), sts


def _check(out, st, want, sts, *, serial=0):
    np.testing.assert_array_equal(out, want)
    assert st.rescale_events == sum(s.rescale_events for s in sts)
    assert st.max_abs_acc == max(s.max_abs_acc for s in sts)
    assert st.max_abs_score == max(s.max_abs_score for s in sts)
    assert st.acc_overflows == sum(s.acc_overflows for s in sts)
    assert st.serial_fallbacks == serial


@pytest.mark.parametrize("T", [1, 2, 63, 64, 65, 1023, 1024, 1025, 3000, 9000])
def test_random_contexts(ctx, T):
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(100 + T)
    k, v = _kv(rng, T)
    c = _cache(ctx, T + 5)
    c.append_rotated(k, v)
    q = rng.integers(-(1 << 22), 1 << 22, size=(32, 64))
    for mode in ("online", "split"):
        out, st = CompressedAttention(c).attend(q[None], mode)
        want, sts = _want(k, v, q, Format())
        _check(out.cpu().numpy()[0], st, want, sts)


def test_both_kernels_agree_on_a_multi_chunk_context(ctx):
    """The same cache through the scan attend, the chunked attend and the serial path."""
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(7)
    T = 5000
    k, v = _kv(rng, T)
    c = _cache(ctx, T)
    c.append_rotated(k, v)
    q = rng.integers(-(1 << 22), 1 << 22, size=(32, 64))
    a = CompressedAttention(c)
    outs = {}
    for pin in ("scan", "chunked"):
        c.pin_kernel(pin)
        outs[pin], st = a.attend(q[None], "online")
        assert st.serial_fallbacks == 0, pin
    outs["serial"], _ = a.attend(q[None], "serial")
    want, _ = _want(k, v, q, Format())
    for name, o in outs.items():
        np.testing.assert_array_equal(o.cpu().numpy()[0], want, err_msg=name)


def test_d128_3b3b(ctx):
    from insitu_amd.attention import CompressedAttention
    f = Format(d=128, key_bits=3, value_bits=3)
    rng = np.random.default_rng(12)
    T = 2600
    k, v = _kv(rng, T, d=128)
    c = _cache(ctx, T, d=128, kb=3, vb=3)
    c.append_rotated(k, v)
    q = rng.integers(-(1 << 22), 1 << 22, size=(32, 128))
    out, st = CompressedAttention(c).attend(q[None], "online")
    want, sts = _want(k, v, q, f)
    _check(out.cpu().numpy()[0], st, want, sts)


@pytest.mark.parametrize("T", [1, 700, 3000, 9000])
def test_eight_query_heads_per_kv_head(ctx, T):
    """n_q = 64 over 8 KV heads (G = 8): the chunked attend does not take it, so the
    automatic choice is the scan attend."""
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(200 + T)
    k, v = _kv(rng, T)
    c = _cache(ctx, T, n_q=64, pin="auto")
    with pytest.raises(Exception):
        c.pin_kernel("chunked")
    c.append_rotated(k, v)
    q = rng.integers(-(1 << 22), 1 << 22, size=(64, 64))
    out, st = CompressedAttention(c).attend(q[None], "online")
    want, sts = _want(k, v, q, Format(), G=8)
    _check(out.cpu().numpy()[0], st, want, sts)


def test_eight_query_heads_ragged_batch(ctx):
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(23)
    lens = [2100, 0, 1, 1025, 4000]
    c = _cache(ctx, max(lens), batch=len(lens), n_q=64, pin="auto")
    data = []
    for b, T in enumerate(lens):
        k, v = _kv(rng, T)
        if T:
            c.append_rotated(k, v, seq=b)
        data.append((k, v))
    q = rng.integers(-(1 << 22), 1 << 22, size=(len(lens), 64, 64))
    out, st = CompressedAttention(c).attend(q, "online")
    out = out.cpu().numpy()
    for b, (k, v) in enumerate(data):
        if lens[b] == 0:
            continue
        want, _ = _want(k, v, q[b], Format(), G=8)
        np.testing.assert_array_equal(out[b], want, err_msg=f"seq {b}")
    assert st.serial_fallbacks == 0


def test_flat_attention_near_the_clamp(ctx):
    """acc climbs towards 0.9 x 2^31 over five chunks without clamping: the replay's
    per-run check passes on the exact accumulator, so no head goes serial."""
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(31)
    T = 4500
    k = rng.integers(-(1 << 16), 1 << 16, size=(T, 8, 64))
    v = 400_000 + rng.integers(-20_000, 20_000, size=(T, 8, 64))
    q = rng.integers(-(1 << 8), 1 << 8, size=(32, 64))
    c = _cache(ctx, T)
    c.append_rotated(k, v)
    out, st = CompressedAttention(c).attend(q[None], "online")
    want, sts = _want(k, v, q, Format())
    _check(out.cpu().numpy()[0], st, want, sts)
    assert st.acc_overflows == 0 and st.max_abs_acc > 0.9 * 2 ** 31


def test_a_clamp_in_a_later_chunk_falls_back_exactly(ctx):
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(31)
    T = 6000
    k = rng.integers(-(1 << 16), 1 << 16, size=(T, 8, 64))
    v = 400_000 + rng.integers(-20_000, 20_000, size=(T, 8, 64))
    q = rng.integers(-(1 << 8), 1 << 8, size=(32, 64))
    c = _cache(ctx, T)
    c.append_rotated(k, v)
    out, st = CompressedAttention(c).attend(q[None], "online")
    want, sts = _want(k, v, q, Format())
    _check(out.cpu().numpy()[0], st, want, sts, serial=32)
    assert st.acc_overflows > 0


def test_rising_scores_overflow_the_runs_and_fall_back_exactly(ctx):
    """Every token a new maximum: a chunk has more runs than it can publish, and the
    heads concerned are recomputed on the serial path, still bit-exact."""
    from insitu_amd.attention import CompressedAttention
    T = 3000
    rng = np.random.default_rng(22)
    base = rng.integers(-(1 << 20), 1 << 20, size=(1, 8, 64))
    grow = np.arange(1, T + 1)[:, None, None] * 1000
    k = np.clip(base + grow * np.sign(base), -(1 << 23), (1 << 23) - 1)
    v = rng.integers(-(1 << 20), 1 << 20, size=(T, 8, 64))
    c = _cache(ctx, T)
    c.append_rotated(k, v)
    q = np.sign(base[0]).repeat(4, axis=0) * (1 << 18)
    out, st = CompressedAttention(c).attend(q[None], "online")
    want, sts = _want(k, v, q, Format())
    np.testing.assert_array_equal(out.cpu().numpy()[0], want)
    assert st.rescale_events == sum(s.rescale_events for s in sts) > 500
    assert st.serial_fallbacks > 0


def test_few_events_in_many_chunks_are_walked_in_order(ctx):
    """Scores that rise slowly across the context: most chunks publish a run opened by
    a rescale event, so the replay applies a factor in almost every chunk."""
    from insitu_amd.attention import CompressedAttention
    T = 40 * 1024
    rng = np.random.default_rng(9)
    base = rng.integers(-(1 << 20), 1 << 20, size=(1, 8, 64))
    step = (np.arange(T) // 700)[:, None, None] * 3000       # equal rows within a block: ties
    k = np.clip(base + step * np.sign(base), -(1 << 23), (1 << 23) - 1)
    v = rng.integers(-(1 << 20), 1 << 20, size=(T, 8, 64))
    c = _cache(ctx, T)
    c.append_rotated(k, v)
    q = np.sign(base[0]).repeat(4, axis=0) * (1 << 12)
    out, st = CompressedAttention(c).attend(q[None], "online")
    want, sts = _want(k, v, q, Format())
    _check(out.cpu().numpy()[0], st, want, sts)
    assert st.rescale_events > 30 * 8


@pytest.mark.parametrize("d,kb,vb", [(64, 4, 2), (128, 3, 3)])
def test_fused_step_ragged_batch(ctx, d, kb, vb):
    """insitu_step through the scan attend: rotate, append and attend in one launch."""
    from insitu_amd import ModelConfig, QuantConfig
    from insitu_amd.block import AttentionBlock
    rng = np.random.default_rng(51 + d)
    lens, steps, batch = [2500, 1100], 3, 2
    model = ModelConfig.llama32_1b() if d == 64 else ModelConfig(
        hidden_size=4096, num_heads=32, num_kv_heads=8, head_dim=128)
    f = Format(d=d, key_bits=kb, value_bits=vb)
    blk = AttentionBlock(model, QuantConfig(key_bits=kb, value_bits=vb),
                         capacity=max(lens) + steps, batch=batch, softmax="online", ctx=ctx)
    blk.cache.pin_kernel("scan")
    sg = signs_from_seed(d, 0, 1)
    hosts = []
    for b, T in enumerate(lens):
        k, v = _kv(rng, T, d=d)
        blk.cache.append_rotated(k, v, seq=b)
        h = Cache(8, T + steps, f)
        h.append_rotated(k, v)
        hosts.append(h)
    for t in range(steps):
        qw = rng.integers(-(1 << 23), 1 << 23, size=(batch, 32, d))
        kw = rng.integers(-(1 << 23), 1 << 23, size=(batch, 8, d))
        vw = rng.integers(-(1 << 23), 1 << 23, size=(batch, 8, d))
        out = blk.step(qw, kw, vw).cpu().numpy().reshape(batch, 32, d)
        for b in range(batch):
            qr, kr, vr = rotate(qw[b], sg), rotate(kw[b], sg), rotate(vw[b], sg)
            hosts[b].append_rotated(kr[None], vr[None])
            want = np.concatenate([native.attend_online(qr[4 * g:4 * g + 4], hosts[b].view(g), f)[0]
                                   for g in range(8)])
            np.testing.assert_array_equal(out[b], want, err_msg=f"step {t} seq {b}")
        assert blk.last_stats.serial_fallbacks == 0 and blk.last_stats.range_errors == 0
    for b, T in enumerate(lens):
        for g in (0, 7):
            np.testing.assert_array_equal(blk.cache.read_rows(g, T, steps, seq=b),
                                          hosts[b].buf[T:T + steps, g])


def test_full_c2_context(ctx):
    """ctx 32,768 on the workload's own distribution (BASELINE config 2's size)."""
    from insitu_amd.attention import CompressedAttention
    from insitu_amd.workload import Workload
    T = 32768
    q, k, v = Workload(seed=0).steps(T)
    sg = signs_from_seed(64, 0, 1)
    kr, vr = rotate(k[0], sg), rotate(v[0], sg)
    qr = rotate(q[0, -1], sg)
    c = _cache(ctx, T)
    c.append_rotated(kr, vr)
    out, st = CompressedAttention(c).attend(qr[None], "online")
    want, sts = _want(kr, vr, qr, Format())
    _check(out.cpu().numpy()[0], st, want, sts)


def test_epoch_words_of_another_kernel_are_not_taken_for_this_ones(ctx):
    """The two kernels share one scratch buffer with different layouts: alternating
    them on one cache re-zeroes the words read before their epoch is checked."""
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(77)
    T = 4100
    k, v = _kv(rng, T)
    c = _cache(ctx, T)
    c.append_rotated(k, v)
    a = CompressedAttention(c)
    want = None
    for i in range(6):
        c.pin_kernel("scan" if i % 2 == 0 else "chunked")
        q = rng.integers(-(1 << 22), 1 << 22, size=(32, 64))
        out, st = a.attend(q[None], "online")
        want, _ = _want(k, v, q, Format())
        np.testing.assert_array_equal(out.cpu().numpy()[0], want, err_msg=f"call {i}")
        assert st.serial_fallbacks == 0
