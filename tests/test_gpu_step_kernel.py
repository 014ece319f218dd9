"""GPU: the decode step's own kernel (attend_step.hip) against the oracle and the chunked attend.

insitu_step (kernel.py:271-345: rotate q/k/v, append the k/v row, attend_online over every
row, finalize) runs on attend_step.hip wherever it handles the cache (d = 64, 4 query heads
per KV head, 4-bit keys, 2-bit values). Each case steps a cache on that kernel and a copy
pinned to the chunked attend's fused step from the same rows, and checks, bit for bit:
  - both outputs against each other and the last one against oracle/c's attend_online
    over the cache's rows (ops/attention.py:451-513);
  - the statistics (attention.py:257-274) of both paths, and that no head fell back to
    the serial path;
  - the appended rows of both caches.
Contexts cover one chunk (1, 2, 64, 65, 100 tokens: the score's channel slices), chunk
edges (1,023-1,025), several chunks, a flat softmax (every token a candidate), a ragged
batch, and the look-back giving up (spin limit 0: every chain with a predecessor goes to
the exact serial path).
"""

import numpy as np
import pytest

from oracle import native
from oracle.quantize import Format
from oracle.rotate import rotate, signs_from_seed

pytestmark = pytest.mark.gpu

N_KV, N_Q, D = 8, 32, 64


def _stats(st):
    return (st.n_tokens, st.rescale_events, st.score_overflows, st.acc_overflows, st.max_abs_score,
            st.max_abs_acc, st.range_errors, st.serial_fallbacks)


def _run(ctx, T, *, steps=2, batch=1, flat=False, seed=0, spin_limit=None, lens=None):
    """Steps two caches (the step kernel, the chunked fused step) from T - 1 rows."""
    import torch
    from insitu_amd import QuantConfig, _lib
    from insitu_amd.cache import CompressedCache
    from insitu_amd.rotate import Rotation
    from insitu_amd.runtime import ptr
    from insitu_amd.workload import Workload

    quant = QuantConfig(key_bits=4, value_bits=2)
    rot = Rotation.for_quant(quant, D)
    wl = Workload(seed=seed)
    _, k, v = wl.steps(T - 1)
    qs, ks, vs = wl.steps(steps)
    if flat:
        qs = qs >> 9                       # small queries: a flat softmax
    kr, vr = rot.apply(k[0], ctx), rot.apply(v[0], ctx)
    lens = lens or [T - 1] * batch
    res = {}
    for path in ("chunked", "step"):
        c = CompressedCache(N_KV, D, T + steps, quant, batch=batch, n_q_heads=N_Q, ctx=ctx)
        for b in range(batch):
            if lens[b] > 0:
                c.append_rotated(kr[:lens[b]], vr[:lens[b]], seq=b)
        c.pin_kernel(path)
        if spin_limit is not None:
            _lib.check(ctx.lib.insitu_cache_debug(c.handle, _lib.DEBUG_SPIN_LIMIT, spin_limit))
        outs, sts = [], []
        for i in range(steps):
            rep = (batch,) + qs[0, i].shape
            qd = ctx.to_device(np.broadcast_to(qs[0, i], rep).copy(), torch.int32)
            kd = ctx.to_device(np.broadcast_to(ks[0, i], (batch,) + ks[0, i].shape).copy(), torch.int32)
            vd = ctx.to_device(np.broadcast_to(vs[0, i], (batch,) + vs[0, i].shape).copy(), torch.int32)
            out = torch.empty((batch, N_Q, D), dtype=torch.int32, device=ctx.torch_device)
            st = _lib.Stats()
            _lib.check(ctx.lib.insitu_step(c.handle, ptr(qd), ptr(kd), ptr(vd), ptr(out), 0, st))
            outs.append(out.cpu().numpy())
            sts.append(_stats(st))
        res[path] = (outs, sts, c)
    return qs, res


def _check(T, qs, res, *, steps=2, batch=1, serial=0, lens=None):
    o1, s1, c1 = res["chunked"]
    o2, s2, c2 = res["step"]
    for a, b in zip(o1, o2):
        np.testing.assert_array_equal(b, a)
    assert s2 == s1
    assert all(s[7] == serial for s in s2), s2
    lens = lens or [T - 1] * batch
    for b in range(batch):
        n = lens[b] + steps
        for h in (0, N_KV - 1):
            np.testing.assert_array_equal(c2.read_rows(h, 0, n, seq=b), c1.read_rows(h, 0, n, seq=b))
    # the oracle over the step kernel's rows, for sequence 0's last step
    sg = signs_from_seed(D, 0, 1)
    qr = rotate(qs[0, steps - 1].astype(np.int64), sg)
    want = np.concatenate([native.attend_online(qr[4 * h:4 * h + 4], c2.view(h), Format())[0]
                           for h in range(N_KV)])
    np.testing.assert_array_equal(o2[-1][0], want)


@pytest.mark.parametrize("T", [1, 2, 64, 65, 100, 300, 1023, 1024, 1025, 1500, 3000, 9000])
def test_step_kernel_contexts(ctx, T):
    qs, res = _run(ctx, T)
    _check(T, qs, res)


@pytest.mark.parametrize("T", [100, 3000])
def test_step_kernel_flat_softmax(ctx, T):
    qs, res = _run(ctx, T, flat=True)
    _check(T, qs, res)


def test_step_kernel_ragged_batch(ctx):
    lens = [2499, 700]
    qs, res = _run(ctx, 2500, batch=2, lens=lens)
    _check(2500, qs, res, batch=2, lens=lens)


def test_step_kernel_lookback_gives_up(ctx):
    # spin limit 0: every chain with a predecessor chunk goes to the exact serial path
    qs, res = _run(ctx, 3000, spin_limit=0, steps=1)
    o1, s1, _ = res["chunked"]
    o2, s2, c2 = res["step"]
    np.testing.assert_array_equal(o2[0], o1[0])
    assert s2[0][7] == N_Q            # every head of every chain
    sg = signs_from_seed(D, 0, 1)
    qr = rotate(qs[0, 0].astype(np.int64), sg)
    want = np.concatenate([native.attend_online(qr[4 * h:4 * h + 4], c2.view(h), Format())[0]
                           for h in range(N_KV)])
    np.testing.assert_array_equal(o2[0][0], want)


def test_step_kernel_is_the_default(ctx):
    # the automatic choice for this format is the step kernel: a cache left on "auto"
    # matches one pinned to it, and the chunked attend's own fused step as well
    import torch
    from insitu_amd import QuantConfig, _lib
    from insitu_amd.cache import CompressedCache
    from insitu_amd.rotate import Rotation
    from insitu_amd.runtime import ptr
    from insitu_amd.workload import Workload

    quant = QuantConfig(key_bits=4, value_bits=2)
    rot = Rotation.for_quant(quant, D)
    wl = Workload(seed=3)
    _, k, v = wl.steps(1999)
    qs, ks, vs = wl.steps(1)
    outs = {}
    for path in ("auto", "step"):
        c = CompressedCache(N_KV, D, 2048, quant, n_q_heads=N_Q, ctx=ctx)
        c.append_rotated(rot.apply(k[0], ctx), rot.apply(v[0], ctx))
        c.pin_kernel(path)
        out = torch.empty((1, N_Q, D), dtype=torch.int32, device=ctx.torch_device)
        qd = ctx.to_device(qs[0, 0][None], torch.int32)
        kd = ctx.to_device(ks[0, 0][None], torch.int32)
        vd = ctx.to_device(vs[0, 0][None], torch.int32)
        _lib.check(ctx.lib.insitu_step(c.handle, ptr(qd), ptr(kd), ptr(vd), ptr(out), 0, None))
        outs[path] = out.cpu().numpy()          # (the inputs stay referenced until this copy)
    np.testing.assert_array_equal(outs["auto"], outs["step"])
