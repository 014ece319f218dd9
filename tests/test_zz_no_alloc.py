"""GPU: insitu_attend_causal_static, the prefill that allocates nothing, against
insitu_attend_causal (which allocates its scratch) and the C oracle.

Two calls in a row on one device, the second with fewer queries and a different
base, so the second reuses the static array the first left behind; then a size
the static array cannot hold is refused before anything runs.
"""

import ctypes

import numpy as np
import pytest

from oracle import native
from oracle.quantize import Cache, Format
from oracle.rotate import rotate, signs_from_seed

pytestmark = pytest.mark.gpu


def _cache(ctx, capacity, *, d=64, kb=4, vb=2, n_kv=8, n_q=32, chunk_tokens=0):
    from insitu_amd import QuantConfig
    from insitu_amd.cache import CompressedCache
    return CompressedCache(n_kv, d, capacity, QuantConfig(key_bits=kb, value_bits=vb),
                           n_q_heads=n_q, chunk_tokens=chunk_tokens, ctx=ctx)


def _static(ctx, c, base, q, mode):
    import torch
    from insitu_amd import _lib
    from insitu_amd.runtime import ptr
    qd = ctx.to_device(q, torch.int32)
    out = torch.empty_like(qd)
    _lib.check(ctx.lib.insitu_attend_causal_static(c.handle, 0, base, int(q.shape[0]), ptr(qd), ptr(out),
                                                   _lib.MODES[mode]))
    return out.cpu().numpy()


@pytest.mark.parametrize("mode", ["online", "two_pass"])
def test_static_prefill_equals_the_allocating_prefill_twice(ctx, mode):
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(23)
    d, T = 64, 2700
    sg = signs_from_seed(d, 0, 1)
    k = rotate(rng.integers(-(1 << 22), 1 << 22, size=(T * 8, d)), sg).reshape(T, 8, d)
    v = rotate(rng.integers(-(1 << 22), 1 << 22, size=(T * 8, d)), sg).reshape(T, 8, d)
    c = _cache(ctx, T)
    c.append_rotated(k, v)
    host = Cache(8, T, Format())
    host.append_rotated(k, v)
    heads = [host.view(h) for h in range(8)]
    a = CompressedAttention(c)
    for call, (base, n_q) in enumerate(((2000, 700), (2400, 90))):
        q = rotate(rng.integers(-(1 << 22), 1 << 22, size=(n_q * 32, d)), sg).reshape(n_q, 32, d)
        want, _ = a.attend_prefill(q, base, mode)
        want = want.cpu().numpy()
        got = _static(ctx, c, base, q, mode)
        np.testing.assert_array_equal(got, want, err_msg=f"call {call}")
        if mode == "online":
            np.testing.assert_array_equal(got, native.decode_steps(q, heads, Format(), base=base),
                                          err_msg=f"call {call} vs the oracle")


def test_static_prefill_refuses_what_its_array_cannot_hold(ctx):
    """64 KV heads at d = 128 over 131,072 rows need about 133 MB of chunk scratch
    for one query, more than the 64 MiB array: EBADLEN, nothing launched."""
    import torch
    from insitu_amd import _lib
    from insitu_amd.runtime import ptr
    c = _cache(ctx, 131072, d=128, kb=3, vb=3, n_kv=64, n_q=256)
    c.set_length(131072)
    q = torch.zeros((1, 256, 128), dtype=torch.int32, device=ctx.torch_device)
    out = torch.empty_like(q)
    rc = ctx.lib.insitu_attend_causal_static(c.handle, 0, 131071, 1, ptr(q), ptr(out), _lib.SEQUENTIAL)
    assert rc == _lib.EBADLEN
    assert b"static scratch" in ctx.lib.insitu_last_error()
