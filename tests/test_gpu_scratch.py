"""GPU: the chunked attend's scratch across attends -- the epoch wrap of each scratch
buffer, and the exits its bounded waits take.

Each cache has two scratch buffers (decode attends, prefill launches), each with its
own attend count; the words an attend publishes carry that count's epoch (1 .. 2^14 - 1),
and at the wrap the buffer is cleared before anything of the attend writes it. A test
hook (insitu_cache_debug) sets the counts next to the wrap and sets the spin limit of
the waits, so both are reached in a few calls. Every output is checked against the C
oracle's online softmax over the same rows.
"""

import ctypes

import numpy as np
import pytest

from oracle import native
from oracle.quantize import Cache, Format
from oracle.rotate import rotate, signs_from_seed

pytestmark = pytest.mark.gpu

WRAP = (1 << 14) - 1


def _block(ctx, d, kb, vb, capacity, softmax="online"):
    from insitu_amd import ModelConfig, QuantConfig
    from insitu_amd.block import AttentionBlock
    model = ModelConfig.llama32_1b() if d == 64 else ModelConfig(
        hidden_size=4096, num_heads=32, num_kv_heads=8, head_dim=128)
    return AttentionBlock(model, QuantConfig(key_bits=kb, value_bits=vb), capacity=capacity,
                          softmax=softmax, ctx=ctx)


def _debug(blk, what, value):
    from insitu_amd import _lib
    _lib.check(blk.ctx.lib.insitu_cache_debug(blk.cache.handle, what, value))


class _Host:
    """The oracle's cache and the wire -> rotated path, kept beside the block's."""

    def __init__(self, d, kb, vb, capacity):
        self.f = Format(d=d, key_bits=kb, value_bits=vb)
        self.sg = signs_from_seed(d, 0, 1)
        self.cache = Cache(8, capacity, self.f)
        self.d = d

    def step_want(self, qw, kw, vw):
        self.cache.append_rotated(rotate(kw, self.sg)[None], rotate(vw, self.sg)[None])
        qr = rotate(qw, self.sg)
        return np.concatenate([native.attend_online(qr[4 * g:4 * g + 4], self.cache.view(g), self.f)[0]
                               for g in range(8)])

    def prefill_want(self, qw, kw, vw):
        base = self.cache.length
        self.cache.append_rotated(rotate(kw.reshape(-1, self.d), self.sg).reshape(kw.shape),
                                  rotate(vw.reshape(-1, self.d), self.sg).reshape(vw.shape))
        qr = rotate(qw.reshape(-1, self.d), self.sg).reshape(qw.shape)
        heads = [self.cache.view(g) for g in range(8)]
        return native.decode_steps(qr, heads, self.f, base=base)


def _wire(rng, n, d):
    return (rng.integers(-(1 << 22), 1 << 22, size=(n, 32, d)),
            rng.integers(-(1 << 22), 1 << 22, size=(n, 8, d)),
            rng.integers(-(1 << 22), 1 << 22, size=(n, 8, d)))


def test_epoch_wrap_of_each_buffer_in_either_order(ctx):
    """A decode step after a prefill at the prefill buffer's wrap, a prefill after a
    decode at the decode buffer's wrap, and steps on either side of each wrap: every
    output exact, no chain sent to the serial path."""
    from insitu_amd import _lib
    rng = np.random.default_rng(11)
    d, T0 = 64, 2600
    blk = _block(ctx, d, 4, 2, T0 + 40)
    host = _Host(d, 4, 2, T0 + 40)
    q, k, v = _wire(rng, T0, d)
    got = blk.prefill(q, k, v).cpu().numpy()
    np.testing.assert_array_equal(got, host.prefill_want(q, k, v).reshape(T0, -1))

    def step(tag):
        qw, kw, vw = _wire(rng, 1, d)
        out = blk.step(qw, kw, vw).cpu().numpy()[0]
        np.testing.assert_array_equal(out, host.step_want(qw[0], kw[0], vw[0]).reshape(-1), err_msg=tag)
        assert blk.last_stats.serial_fallbacks == 0, tag

    def prefill(tag, n=5):
        qw, kw, vw = _wire(rng, n, d)
        out = blk.prefill(qw, kw, vw).cpu().numpy()
        np.testing.assert_array_equal(out, host.prefill_want(qw, kw, vw).reshape(n, -1), err_msg=tag)
        assert blk.last_stats.serial_fallbacks == 0, tag

    # the prefill buffer wraps on its next launch; decode steps follow
    _debug(blk, _lib.DEBUG_PREFILL_CALLS, WRAP - 1)
    prefill("prefill before the wrap")          # epoch 2^14 - 1
    prefill("prefill at the wrap")              # cleared, epoch 1
    step("decode after a prefill at the wrap")
    step("decode again")
    # the decode buffer wraps; a prefill follows, then more steps
    _debug(blk, _lib.DEBUG_DECODE_CALLS, WRAP - 1)
    step("decode before the wrap")
    step("decode at the wrap")
    prefill("prefill after a decode at the wrap")
    step("decode after the wrap")
    step("decode after the wrap, again")


def test_epoch_wrap_keeps_the_staged_queries_of_a_two_launch_step(ctx):
    """At d = 128 a decode step is two launches: a write kernel stages the rotated
    queries in the decode scratch, then the attend. The wrap's clear comes before the
    staging, so the step at the wrap is exact on the chunked path (no serial chains)."""
    from insitu_amd import _lib
    rng = np.random.default_rng(13)
    d, T0 = 128, 2100
    blk = _block(ctx, d, 3, 3, T0 + 8)
    host = _Host(d, 3, 3, T0 + 8)
    k = rng.integers(-(1 << 22), 1 << 22, size=(T0, 8, d))
    v = rng.integers(-(1 << 22), 1 << 22, size=(T0, 8, d))
    kr = rotate(k.reshape(-1, d), host.sg).reshape(T0, 8, d)
    vr = rotate(v.reshape(-1, d), host.sg).reshape(T0, 8, d)
    blk.cache.append_rotated(kr, vr)
    host.cache.append_rotated(kr, vr)
    _debug(blk, _lib.DEBUG_DECODE_CALLS, WRAP - 1)
    for tag in ("before the wrap", "at the wrap", "after the wrap"):
        qw, kw, vw = _wire(rng, 1, d)
        out = blk.step(qw, kw, vw).cpu().numpy()[0]
        np.testing.assert_array_equal(out, host.step_want(qw[0], kw[0], vw[0]).reshape(-1), err_msg=tag)
        assert blk.last_stats.serial_fallbacks == 0, tag


@pytest.mark.parametrize("path", ["step", "attend", "prefill"])
def test_waits_that_give_up_send_the_chain_to_the_exact_serial_path(ctx, path):
    """With the spin limit at 0 every wait on another workgroup gives up at once
    (the exit a stalled predecessor would take): the output is still exact, through
    the serial path, and each chain that needed a predecessor is counted."""
    from insitu_amd import _lib
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(17)
    d, T0 = 64, 2500
    blk = _block(ctx, d, 4, 2, T0 + 4)
    host = _Host(d, 4, 2, T0 + 4)
    k = rng.integers(-(1 << 22), 1 << 22, size=(T0, 8, d))
    v = rng.integers(-(1 << 22), 1 << 22, size=(T0, 8, d))
    kr = rotate(k.reshape(-1, d), host.sg).reshape(T0, 8, d)
    vr = rotate(v.reshape(-1, d), host.sg).reshape(T0, 8, d)
    blk.cache.append_rotated(kr, vr)
    host.cache.append_rotated(kr, vr)
    _debug(blk, _lib.DEBUG_SPIN_LIMIT, 0)
    try:
        if path == "step":
            qw, kw, vw = _wire(rng, 1, d)
            out = blk.step(qw, kw, vw).cpu().numpy()[0]
            want = host.step_want(qw[0], kw[0], vw[0]).reshape(-1)
            st = blk.last_stats
            n_chains = 8
        elif path == "attend":
            qr = rotate(rng.integers(-(1 << 22), 1 << 22, size=(32, d)), host.sg)
            o, st = CompressedAttention(blk.cache).attend(qr[None], "online")
            out = o.cpu().numpy()[0].reshape(-1)
            want = np.concatenate([native.attend_online(qr[4 * g:4 * g + 4], host.cache.view(g), host.f)[0]
                                   for g in range(8)]).reshape(-1)
            n_chains = 8
        else:
            qw, kw, vw = _wire(rng, 3, d)
            out = blk.prefill(qw, kw, vw).cpu().numpy()
            want = host.prefill_want(qw, kw, vw).reshape(3, -1)
            st = blk.last_stats
            n_chains = 3 * 8
        np.testing.assert_array_equal(out, want)
        # every chain spans 3 chunks, so every chain has a wait that gave up
        assert st.serial_fallbacks == n_chains * 4
    finally:
        _debug(blk, _lib.DEBUG_SPIN_LIMIT, 1 << 20)
    # and with the limit restored the same cache attends on the chunked path again
    qw, kw, vw = _wire(rng, 1, d)
    out = blk.step(qw, kw, vw).cpu().numpy()[0]
    np.testing.assert_array_equal(out, host.step_want(qw[0], kw[0], vw[0]).reshape(-1))
    assert blk.last_stats.serial_fallbacks == 0
