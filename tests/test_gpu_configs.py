"""GPU: the benchmark configurations at their full shapes, against oracle/c.

C3  batch 64, one Llama-3.2-1B-shape layer (32 q heads, 8 KV heads, d = 64, 4b K / 2b V),
    context lengths uniform in [1024, 8192] from seed 3; each sequence its own seeded
    k/v and query; one attend launch over the whole batch. Every sequence and KV group
    against attend_online on the device's rows, and the rows of four sequences against
    the oracle's encode + pack of the same rotated k/v.
C4  Llama-3-8B shape (32 q heads, 8 KV heads, d = 128, 3b K / 3b V), batch 16, ctx 131,072,
    one layer (a 1.68 GB compressed cache). The k/v (2.1 G values each) are drawn on the
    GPU (torch.Generator, seed per sequence) from the configuration's distribution:
    N(0, 1) with 1 % of channels per head scaled x16, cast to Q8.16 (rint, 24-bit
    saturation), then rotated and appended. Every sequence against oracle/c on two KV
    heads, all eight heads of one sequence, and a sample of rows of every sequence
    against the oracle's encode + pack.
C1  16 layers x 4,096 sequential decode steps from an empty cache (insitu_step: rotate,
    append, attend), every step's output and every cache byte against oracle/c.

The oracle runs on the host in threads (its C calls release the GIL).
"""

import concurrent.futures
import os

import numpy as np
import pytest

from insitu_amd.cache import unpack_rows
from oracle import native
from oracle.quantize import Format, encode, pack
from oracle.rotate import rotate, signs_from_seed

pytestmark = pytest.mark.gpu

WORKERS = max(1, min(16, len(os.sched_getaffinity(0))))


def _pool():
    return concurrent.futures.ThreadPoolExecutor(max_workers=WORKERS)


def test_c3_batch64_ragged_every_sequence_and_group(ctx):
    from insitu_amd import QuantConfig
    from insitu_amd.attention import CompressedAttention
    from insitu_amd.cache import CompressedCache
    from insitu_amd.rotate import Rotation
    from insitu_amd.workload import fill_ragged
    d, batch = 64, 64
    f = Format()
    lens = np.random.default_rng(3).integers(1024, 8193, size=batch)
    quant = QuantConfig(key_bits=4, value_bits=2)
    rot = Rotation.for_quant(quant, d)
    c = CompressedCache(8, d, int(lens.max()), quant, batch=batch, n_q_heads=32, ctx=ctx)
    q, kept = fill_ragged(c, lens, 3000, rot, ctx, keep=(5, 21, 37, 53))
    assert c.lengths() == [int(x) for x in lens]
    out, st = CompressedAttention(c).attend(q, "online")
    out = out.cpu().numpy()
    assert st.serial_fallbacks == 0

    # the device rows are read on this thread (a cache handle is not thread-safe);
    # decoding them and the oracle run in the pool
    rows = {(b, h): c.read_rows(h, 0, None, b) for b in range(batch) for h in range(8)}

    def check(bh):
        b, h = bh
        kv = unpack_rows(rows[bh], d, 4, 2)
        want, _ = native.attend_online(q[b, 4 * h:4 * h + 4], kv, f)
        return bh, bool(np.array_equal(out[b, 4 * h:4 * h + 4], want))

    with _pool() as ex:
        results = list(ex.map(check, rows))
    assert all(ok for _, ok in results), [bh for bh, ok in results if not ok]
    for b, (kr, vr) in kept.items():
        for h in (0, 3, 7):
            np.testing.assert_array_equal(rows[(b, h)], pack(encode(kr[:, h], vr[:, h], f), f),
                                          err_msg=f"rows of sequence {b}, KV head {h}")


def test_c4_one_layer_full_shape(ctx):
    from insitu_amd import QuantConfig
    from insitu_amd.attention import CompressedAttention
    from insitu_amd.cache import CompressedCache
    from insitu_amd.rotate import Rotation
    from insitu_amd.workload import fill_on_device
    d, batch, T = 128, 16, 131072
    f = Format(d=128, key_bits=3, value_bits=3)
    quant = QuantConfig(key_bits=3, value_bits=3)
    rot = Rotation.for_quant(quant, d)
    c = CompressedCache(8, d, T, quant, batch=batch, n_q_heads=32, ctx=ctx)
    q, samples = fill_on_device(c, T, 4000, rot, ctx, sample_rows=8)
    print("c4: cache filled", flush=True)
    assert c.lengths() == [T] * batch
    out, st = CompressedAttention(c).attend(q, "online")
    out = out.cpu().numpy()
    assert st.serial_fallbacks == 0 and st.n_tokens == T
    groups = [(b, h) for b in range(batch) for h in (0, 5)] + [(7, h) for h in (1, 2, 3, 4, 6, 7)]
    rows = {bh: c.read_rows(bh[1], 0, None, bh[0]) for bh in groups}

    def check(bh):
        b, h = bh
        kv = unpack_rows(rows[bh], d, 3, 3)
        want, _ = native.attend_online(q[b, 4 * h:4 * h + 4], kv, f)
        return bh, bool(np.array_equal(out[b, 4 * h:4 * h + 4], want))

    with _pool() as ex:
        results = list(ex.map(check, groups))
    assert all(ok for _, ok in results), [bh for bh, ok in results if not ok]
    assert len(samples) == batch
    for b, (ts, kr, vr) in samples.items():
        for h in (0, 6):
            got = np.stack([c.read_rows(h, int(t), 1, b)[0] for t in ts])
            np.testing.assert_array_equal(got, pack(encode(kr[:, h], vr[:, h], f), f),
                                          err_msg=f"sampled rows of sequence {b}, KV head {h}")


def test_c1_full_every_step_and_every_cache_byte(ctx):
    """16 layers x 4,096 steps from empty; layer l draws its q/k/v from Workload(seed
    1000 + l), as bench.py --config c1 does. Each step is one insitu_step per layer."""
    import torch
    from insitu_amd import QuantConfig, _lib
    from insitu_amd.cache import CompressedCache
    from insitu_amd.runtime import ptr
    from insitu_amd.workload import Workload
    L, S, d = 16, 4096, 64
    f = Format()
    quant = QuantConfig(key_bits=4, value_bits=2)
    wire = [Workload(seed=1000 + l).steps(S) for l in range(L)]
    caches = [CompressedCache(8, d, S, quant, ctx=ctx) for _ in range(L)]
    dev = [tuple(ctx.to_device(x[0], torch.int32) for x in w) for w in wire]
    outs = torch.empty((L, S, 32, d), dtype=torch.int32, device=ctx.torch_device)
    lib = ctx.lib
    for t in range(S):
        for l in range(L):
            qd, kd, vd = dev[l]
            _lib.check(lib.insitu_step(caches[l].handle, ptr(qd[t]), ptr(kd[t]), ptr(vd[t]),
                                       ptr(outs[l, t]), _lib.MODES["online"], None))
        if t % 1024 == 1023:
            torch.cuda.synchronize()
            print(f"c1: {t + 1} of {S} steps", flush=True)
    got = outs.cpu().numpy()
    bufs = [c.buf for c in caches]
    sg = signs_from_seed(d, 0, 1)

    def check(l):
        q, k, v = (np.asarray(x[0], dtype=np.int64) for x in wire[l])
        qr = rotate(q.reshape(-1, d), sg).reshape(S, 32, d)
        kr = rotate(k.reshape(-1, d), sg).reshape(S, 8, d)
        vr = rotate(v.reshape(-1, d), sg).reshape(S, 8, d)
        heads = [encode(kr[:, h], vr[:, h], f) for h in range(8)]
        want = native.decode_steps(qr, heads, f)
        bad = np.nonzero((got[l] != want).reshape(S, -1).any(axis=1))[0]
        rows = np.stack([pack(hd, f) for hd in heads], axis=1)
        return l, bad[:5].tolist(), bool(np.array_equal(bufs[l][:S], rows))

    with _pool() as ex:
        results = list(ex.map(check, range(L)))
    assert all(not bad for _, bad, _ in results), {l: bad for l, bad, _ in results if bad}
    assert all(ok for _, _, ok in results), [l for l, _, ok in results if not ok]
