"""GPU parity: every stage of the HIP path against the oracle and the reference's goldens.

All calls go through libinsitu_hip.so (the C ABI). Bit-exact is the bar for
every integer stage. Sizes are chosen so the oracle finishes in seconds.
"""

import numpy as np
import pytest

from oracle import hexio as hx
from oracle import native
from oracle.attention import attend_online, attend_two_pass
from oracle.layout import DdrLayout
from oracle.quantize import Cache, Format, encode, pack, unpack
from oracle.rotate import rotate, signs_from_seed

pytestmark = pytest.mark.gpu

FMT = Format()


def _cache(ctx, capacity, *, d=64, kb=4, vb=2, batch=1, n_kv=8, n_q=32, chunk_tokens=0):
    from insitu_amd import QuantConfig
    from insitu_amd.cache import CompressedCache
    return CompressedCache(n_kv, d, capacity, QuantConfig(key_bits=kb, value_bits=vb),
                           batch=batch, n_q_heads=n_q, chunk_tokens=chunk_tokens, ctx=ctx)


@pytest.fixture(scope="module")
def fixture_cache(ctx):
    rows = np.stack([hx.bytes_rows(f"cache_rows_h{h}.hex") for h in range(8)], axis=1)
    c = _cache(ctx, 65)
    for h in range(8):
        c.load_rows(rows[:, h], h)
    c.set_length(65)
    return c, rows


# -- the write path -----------------------------------------------------------

def test_rotation_random_vectors_and_wire(ctx):
    from insitu_amd.rotate import Rotation
    rot = Rotation.from_seed(64, 0, 1)
    assert rot.sign_words()[0][0] == 0x81191FF5899001F8
    rin = hx.lanes("rot_random_in.hex", 24, 64)
    got = rot.apply(rin, ctx).cpu().numpy()
    np.testing.assert_array_equal(got, hx.lanes("rot_random_out.hex", 24, 64))
    for n in "qkv":
        got = rot.apply(hx.lanes(f"wire_{n}.hex", 24, 64), ctx).cpu().numpy()
        np.testing.assert_array_equal(got, hx.lanes(f"rot_{n}.hex", 24, 64))


@pytest.mark.parametrize("d,rounds,seed", [(128, 1, 0), (64, 2, 3), (128, 2, 5), (64, 0, 0)])
def test_rotation_other_shapes_against_oracle(ctx, d, rounds, seed):
    from insitu_amd.rotate import Rotation
    rng = np.random.default_rng(d + rounds)
    x = rng.integers(-(1 << 23), 1 << 23, size=(300, d))
    rot = Rotation.from_seed(d, seed, rounds)
    np.testing.assert_array_equal(rot.apply(x, ctx).cpu().numpy(),
                                  rotate(x, signs_from_seed(d, seed, rounds)))


def test_encoder_norms_and_codes_including_ties(ctx):
    from insitu_amd import ops
    x = hx.lanes("enc_in.hex", 24, 64)
    _, kb, _, vb = FMT.codebooks()
    for bits, bnd, name in ((4, kb, "key"), (2, vb, "value")):
        norm, codes = ops.encode(x, bnd, bits, ctx=ctx)
        np.testing.assert_array_equal(norm, hx.scalars("enc_norm.hex", 16))
        np.testing.assert_array_equal(codes, hx.lanes(f"enc_idx_{name}.hex", 8, 64, signed=False))


def test_qtab(ctx):
    from insitu_amd import ops
    rq = hx.lanes("rot_q.hex", 24, 64)
    got = ops.qtab(rq, FMT.codebooks()[0], ctx)
    np.testing.assert_array_equal(got.reshape(32, -1), hx.lanes("qtab_table.hex", 43, 64 * 16))


def test_exp_lut_every_reachable_output(ctx):
    from insitu_amd import ops
    d = hx.scalars("exp_in.hex", 48)
    np.testing.assert_array_equal(ops.exp_lut(d, ctx), hx.scalars("exp_out.hex", 16, signed=False))
    with pytest.raises(ValueError):
        ops.exp_lut(np.array([-1]), ctx)


def test_finalize_goldens(ctx):
    from insitu_amd import ops
    fa, fl = hx.lanes("fin_acc.hex", 32, 64), hx.scalars("fin_l.hex", 48)
    out, r, sh = ops.finalize(fa, fl, ctx)
    np.testing.assert_array_equal(r, hx.scalars("fin_recip.hex", 32, signed=False))
    np.testing.assert_array_equal(sh, hx.scalars("fin_shift.hex", 8, signed=False))
    np.testing.assert_array_equal(out, hx.lanes("fin_out.hex", 48, 64))


def test_finalize_reciprocal_edges(ctx):
    """l across its whole 48-bit range, powers of two and their neighbours, and
    denominators whose 2^62 / l_n quotient sits just below an integer."""
    from insitu_amd import ops
    from oracle.attention import finalize, reciprocal
    fmt = Format()
    rng = np.random.default_rng(7)
    edges = [1, 2, 3, (1 << 31) - 1, 1 << 31, (1 << 31) + 1, (1 << 32) - 1, 1 << 32,
             (1 << 47) - 1, 1 << 47, (1 << 48) - 1]
    pows = [x for b in range(1, 48) for x in ((1 << b) - 1, 1 << b, (1 << b) + 1)]
    ln = rng.integers(1 << 31, 1 << 32, size=4000, dtype=np.int64)
    near = ((1 << 62) // ((1 << 62) // ln + 1)) + 1     # quotient just below an integer
    ls = np.concatenate([edges, pows, rng.integers(1, 1 << 48, size=2000), near]).astype(np.int64)
    acc = rng.integers(-(1 << 31), 1 << 31, size=(ls.size, 8)).astype(np.int64)
    out, r, sh = ops.finalize(acc, ls, ctx)
    want_r, want_sh = reciprocal(ls, fmt)
    np.testing.assert_array_equal(r, want_r)
    np.testing.assert_array_equal(sh, want_sh)
    np.testing.assert_array_equal(out, finalize(acc, ls, fmt))


def test_append_writes_kv_rows(ctx):
    c = _cache(ctx, 4)
    rk, rv = hx.lanes("rot_k.hex", 24, 64), hx.lanes("rot_v.hex", 24, 64)
    c.append_rotated(rk[None], rv[None])
    assert c.length == 1
    np.testing.assert_array_equal(c.buf[0], hx.bytes_rows("kv_rows.hex"))


@pytest.mark.parametrize("d,kb,vb", [(64, 4, 2), (128, 3, 3), (64, 1, 8), (128, 5, 2)])
def test_append_matches_oracle_encode_pack(ctx, d, kb, vb):
    f = Format(d=d, key_bits=kb, value_bits=vb)
    rng = np.random.default_rng(kb * 10 + vb)
    n = 37
    k = rng.integers(-(1 << 23), 1 << 23, size=(n, 8, d))
    v = rng.integers(-(1 << 23), 1 << 23, size=(n, 8, d))
    k[3, 2] = 0                                   # zero vector: norm 0, all-equal codes
    c = _cache(ctx, 64, d=d, kb=kb, vb=vb)
    c.append_rotated(k[:20], v[:20])
    c.append_rotated(k[20:], v[20:])
    assert c.length == n
    np.testing.assert_array_equal(c.buf, pack(encode(k, v, f), f))
    with pytest.raises(ValueError):
        c.append_rotated(k, v)                     # 37 + 37 > 64 (base.py:67-73)
    assert c.length == n


def test_device_plane_image_is_the_ddr_image(fixture_cache):
    c, rows = fixture_cache
    lay = DdrLayout.for_format(FMT, 8, 65)
    assert {k: v for k, v in c.layout().items() if k in lay.describe()} == lay.describe()
    np.testing.assert_array_equal(c.image(), hx.bytes_rows("ddr_image.hex").reshape(-1))
    np.testing.assert_array_equal(c.buf, rows)


# -- attention ------------------------------------------------------------------

@pytest.mark.parametrize("mode", ["online", "serial", "split"])
def test_out_online_golden(fixture_cache, mode):
    from insitu_amd.attention import CompressedAttention
    c, _ = fixture_cache
    q = hx.lanes("rot_q.hex", 24, 64)
    out, st = CompressedAttention(c).attend(q[None], mode)
    np.testing.assert_array_equal(out.cpu().numpy().reshape(-1),
                                  hx.lanes("out.online.hex", 24, 2048)[0])
    assert st.n_tokens == 65 and st.acc_overflows == 0 and st.score_overflows == 0


def test_out_two_pass_golden(fixture_cache):
    from insitu_amd.attention import CompressedAttention
    c, _ = fixture_cache
    q = hx.lanes("rot_q.hex", 24, 64)
    out, st = CompressedAttention(c).attend(q[None], "two_pass")
    np.testing.assert_array_equal(out.cpu().numpy().reshape(-1), hx.lanes("out.hex", 24, 2048)[0])
    assert st.rescale_events == 0


def test_signed_norm_edge_rows_on_the_device(ctx):
    """score_edge_rows.hex: five rows whose signed key norms are 0, 1, 2^15 - 1, -2^15 and
    -1, which only a loaded image can hold (the encoder never writes them). Loaded with
    load_rows into KV head 0 and attended by the device: alone, each row's |score|
    comes back as max_abs_score and equals score_edge_gold.hex (the reference's scores
    of those rows against rot_q[0]); all five together give the oracle's attend_online
    output and statistics, on both sequential kernels."""
    from insitu_amd.attention import CompressedAttention
    rows = hx.bytes_rows("score_edge_rows.hex")
    gold = hx.scalars("score_edge_gold.hex", 48)
    rq = hx.lanes("rot_q.hex", 24, 64)
    assert list(unpack(rows, FMT).k_norm) == [0, 1, 32767, -32768, -1]
    q = np.zeros((1, 32, 64), dtype=np.int64)
    q[0, 0] = rq[0]                      # the only nonzero query: head 0, KV group 0
    for i in range(5):
        c = _cache(ctx, 5)
        c.load_rows(rows[i:i + 1], 0)
        c.set_length(1)
        for mode in ("serial", "online"):
            _, st = CompressedAttention(c).attend(q, mode)
            assert st.max_abs_score == abs(int(gold[i])), f"row {i}, {mode}"
        one = unpack(rows[i:i + 1], FMT)
        _, hst = CompressedAttention(c).attend_online(rq[0:4], c.view(0))
        assert hst.max_abs_score == int(np.abs(native.scores(rq[0:4], one, FMT)[0]).max())
    c = _cache(ctx, 5)
    c.load_rows(rows, 0)
    c.set_length(5)
    want, wst = attend_online(rq[:4], unpack(rows, FMT), FMT)
    got, st = CompressedAttention(c).attend_online(rq[:4], c.view(0))      # the per-head entry
    np.testing.assert_array_equal(got, want)
    assert (st.max_abs_score, st.rescale_events, st.max_abs_acc) == \
        (wst.max_abs_score, wst.rescale_events, wst.max_abs_acc)
    q4 = np.zeros((1, 32, 64), dtype=np.int64)
    q4[0, :4] = rq[:4]
    for pin in ("scan", "chunked"):                                            # the whole-cache attend
        c.pin_kernel(pin)
        out, st = CompressedAttention(c).attend(q4, "online")
        np.testing.assert_array_equal(out.cpu().numpy()[0, :4], want, err_msg=pin)
        assert st.max_abs_score == wst.max_abs_score, pin
    assert wst.max_abs_score >= max(abs(int(x)) for x in gold)


def test_stress_query_group0_matches_oracle_stats(fixture_cache):
    from insitu_amd.attention import CompressedAttention
    c, rows = fixture_cache
    q2 = hx.lanes("sm2_q.hex", 24, 64)
    got, st = CompressedAttention(c).attend_online(q2, 0)
    want, wst = attend_online(q2, unpack(rows[:, 0], FMT), FMT)
    np.testing.assert_array_equal(got, want)


def _random_cache_inputs(rng, T, d=64, n_kv=8, scale=1 << 20):
    k = rng.integers(-scale, scale, size=(T, n_kv, d))
    v = rng.integers(-scale, scale, size=(T, n_kv, d))
    return k, v


@pytest.mark.parametrize("mode", ["online", "two_pass", "split"])
@pytest.mark.parametrize("T", [1, 2, 63, 64, 65, 700, 3000])
def test_attend_random_contexts_against_native_oracle(ctx, mode, T):
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(T)
    k, v = _random_cache_inputs(rng, T)
    c = _cache(ctx, T + 5)
    c.append_rotated(k, v)
    q = rng.integers(-(1 << 22), 1 << 22, size=(32, 64))
    out, st = CompressedAttention(c).attend(q[None], mode)
    host = Cache(8, T, FMT)
    host.append_rotated(k, v)
    fn = native.attend_two_pass if mode == "two_pass" else native.attend_online
    want = np.concatenate([fn(q[4 * h:4 * h + 4], host.view(h), FMT)[0] for h in range(8)])
    np.testing.assert_array_equal(out.cpu().numpy()[0], want)


def test_acc_clamp_path_is_exact(ctx):
    """Huge value norms drive the int32 accumulator into its clamp; the online path clamps
    per token (attention.py:502-503), two-pass once at the end (:443-444)."""
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(11)
    T = 1000
    k = rng.integers(-(1 << 16), 1 << 16, size=(T, 8, 64))          # flat attention
    v = rng.integers(-(1 << 23), 1 << 23, size=(T, 8, 64))
    v[:, :, :] = np.abs(v[:, :, :])                                 # same-sign channels pile up
    c = _cache(ctx, T)
    c.append_rotated(k, v)
    q = rng.integers(-(1 << 10), 1 << 10, size=(32, 64))
    host = Cache(8, T, FMT)
    host.append_rotated(k, v)
    for mode, fn in (("online", native.attend_online), ("two_pass", native.attend_two_pass)):
        out, st = CompressedAttention(c).attend(q[None], mode)
        want, sts = [], []
        for h in range(8):
            o, s = fn(q[4 * h:4 * h + 4], host.view(h), FMT)
            want.append(o)
            sts.append(s)
        np.testing.assert_array_equal(out.cpu().numpy()[0], np.concatenate(want))
        assert st.acc_overflows == sum(s.acc_overflows for s in sts)
        assert st.acc_overflows > 0, "the case must actually reach the clamp"
        if mode == "online":
            assert st.serial_fallbacks > 0, "the accumulator bound must have sent heads to the serial path"
        assert st.rescale_events == sum(s.rescale_events for s in sts)
        assert st.max_abs_acc == max(s.max_abs_acc for s in sts)
        assert st.max_abs_score == max(s.max_abs_score for s in sts)


def _flat_cache(ctx, T, seed=31):
    """Flat attention (small q and k: every p near 2^15) over same-sign values, so acc
    climbs about 465,000 per token towards the int32 clamp, across several chunks."""
    rng = np.random.default_rng(seed)
    k = rng.integers(-(1 << 16), 1 << 16, size=(T, 8, 64))
    v = 400_000 + rng.integers(-20_000, 20_000, size=(T, 8, 64))
    q = rng.integers(-(1 << 8), 1 << 8, size=(32, 64))
    c = _cache(ctx, T)
    c.append_rotated(k, v)
    host = Cache(8, T, FMT)
    host.append_rotated(k, v)
    return c, host, q


def _online_against_oracle(c, host, q):
    from insitu_amd.attention import CompressedAttention
    out, st = CompressedAttention(c).attend(q[None], "online")
    want, sts = [], []
    for h in range(8):
        o, s = native.attend_online(q[4 * h:4 * h + 4], host.view(h), FMT)
        want.append(o)
        sts.append(s)
    np.testing.assert_array_equal(out.cpu().numpy()[0], np.concatenate(want))
    assert st.acc_overflows == sum(s.acc_overflows for s in sts)
    assert st.rescale_events == sum(s.rescale_events for s in sts)
    assert st.max_abs_acc == max(s.max_abs_acc for s in sts)
    return st


def test_flat_attention_near_the_clamp_stays_on_the_chunked_path(ctx):
    """acc reaches 0.9 x 2^31 in the fifth chunk without clamping: the runs' measured
    prefix sums certify it, so no head needs the serial path (a sum of |terms| bound
    would not)."""
    c, host, q = _flat_cache(ctx, 4500)
    st = _online_against_oracle(c, host, q)
    assert st.acc_overflows == 0 and st.max_abs_acc > 0.9 * 2 ** 31
    assert st.serial_fallbacks == 0


def test_a_clamp_in_a_later_chunk_falls_back_exactly(ctx):
    """The clamp first fires past token 4,600 (chunk 4): the replay's per-run check
    sends every head to the serial path, which clamps token by token."""
    c, host, q = _flat_cache(ctx, 6000)
    st = _online_against_oracle(c, host, q)
    assert st.acc_overflows > 0 and st.serial_fallbacks == 32


def test_small_queries_over_a_long_context_need_no_serial_path(ctx):
    """Projections of small hidden states: |q| < 2^9 against the workload's keys and
    values over 9,000 tokens, a nearly uniform softmax."""
    from insitu_amd.workload import Workload
    from insitu_amd.rotate import Rotation
    T = 9000
    _, k, v = Workload(seed=5).steps(T)
    rot = Rotation.from_seed(64, 0, 1)
    kr = rot.apply(k[0], ctx).cpu().numpy()
    vr = rot.apply(v[0], ctx).cpu().numpy()
    c = _cache(ctx, T)
    c.append_rotated(kr, vr)
    host = Cache(8, T, FMT)
    host.append_rotated(kr, vr)
    q = np.random.default_rng(6).integers(-(1 << 9), 1 << 9, size=(32, 64))
    st = _online_against_oracle(c, host, q)
    assert st.serial_fallbacks == 0


def test_d128_3b3b_against_native_oracle(ctx):
    from insitu_amd.attention import CompressedAttention
    f = Format(d=128, key_bits=3, value_bits=3)
    rng = np.random.default_rng(12)
    T = 500
    k, v = _random_cache_inputs(rng, T, d=128)
    c = _cache(ctx, T, d=128, kb=3, vb=3)
    c.append_rotated(k, v)
    q = rng.integers(-(1 << 22), 1 << 22, size=(32, 128))
    host = Cache(8, T, f)
    host.append_rotated(k, v)
    for mode, fn in (("online", native.attend_online), ("two_pass", native.attend_two_pass)):
        out, _ = CompressedAttention(c).attend(q[None], mode)
        want = np.concatenate([fn(q[4 * h:4 * h + 4], host.view(h), f)[0] for h in range(8)])
        np.testing.assert_array_equal(out.cpu().numpy()[0], want)


def test_batched_ragged_sequences(ctx):
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(13)
    lens = [1, 130, 64, 257]
    c = _cache(ctx, 300, batch=len(lens))
    hosts = []
    for b, T in enumerate(lens):
        k, v = _random_cache_inputs(rng, T)
        c.append_rotated(k, v, seq=b)
        h = Cache(8, T, FMT)
        h.append_rotated(k, v)
        hosts.append(h)
    assert c.lengths() == lens
    q = rng.integers(-(1 << 22), 1 << 22, size=(len(lens), 32, 64))
    out, _ = CompressedAttention(c).attend(q, "online")
    out = out.cpu().numpy()
    for b, h in enumerate(hosts):
        want = np.concatenate([native.attend_online(q[b, 4 * g:4 * g + 4], h.view(g), FMT)[0]
                               for g in range(8)])
        np.testing.assert_array_equal(out[b], want)


# -- the seam: sequential decode from an empty cache ------------------------------

def test_sequential_decode_from_empty_matches_the_oracle_every_step(ctx):
    """Config-1 shape at reduced length: every step appends then attends (kernel.py:253-353)."""
    from insitu_amd import ModelConfig, QuantConfig
    from insitu_amd.block import AttentionBlock
    from insitu_amd.workload import Workload
    steps = 48
    wl = Workload(seed=0)
    qi, ki, vi = wl.steps(steps)
    blk = AttentionBlock(ModelConfig.llama32_1b(), QuantConfig(key_bits=4, value_bits=2),
                         capacity=steps, ctx=ctx)
    sg = signs_from_seed(64, 0, 1)
    host = Cache(8, steps, FMT)
    for t in range(steps):
        out = blk.step(qi[:, t], ki[:, t], vi[:, t]).cpu().numpy()[0]
        qr, kr, vr = rotate(qi[0, t], sg), rotate(ki[0, t], sg), rotate(vi[0, t], sg)
        host.append_rotated(kr[None], vr[None])
        want = np.concatenate([attend_online(qr[4 * h:4 * h + 4], host.view(h), FMT)[0]
                               for h in range(8)]).reshape(-1)
        np.testing.assert_array_equal(out, want, err_msg=f"step {t}")
    np.testing.assert_array_equal(blk.cache.buf, host.buf[:steps])


def test_config0_one_decode_step_at_ctx_512(ctx):
    """Config 0 exactly: Llama-3.2-1B shape, seed 0, 511 cached tokens, then one
    decode step (rotate, append, attend) at context 512, against the numpy
    per-token loop over all 8 KV groups."""
    from insitu_amd import ModelConfig, QuantConfig
    from insitu_amd.block import AttentionBlock
    from insitu_amd.workload import Workload

    n = 512
    q, k, v = Workload(seed=0).steps(n)
    blk = AttentionBlock(ModelConfig.llama32_1b(), QuantConfig(key_bits=4, value_bits=2),
                         capacity=n, ctx=ctx)
    sg = signs_from_seed(64, 0, 1)
    kr, vr = rotate(k[0], sg), rotate(v[0], sg)
    blk.cache.append_rotated(kr[:n - 1], vr[:n - 1])
    out = blk.step(q[:, n - 1], k[:, n - 1], v[:, n - 1]).cpu().numpy()[0]
    host = Cache(8, n, FMT)
    host.append_rotated(kr, vr)
    qr = rotate(q[0, n - 1], sg)
    want = np.concatenate([attend_online(qr[4 * h:4 * h + 4], host.view(h), FMT)[0]
                           for h in range(8)]).reshape(-1)
    np.testing.assert_array_equal(out, want)
    np.testing.assert_array_equal(blk.cache.buf, host.buf)


@pytest.mark.parametrize("mode", ["online", "two_pass"])
def test_config1_layers_from_empty_every_step_and_every_cache_byte(ctx, mode):
    """Config 1 at reduced size: 2 layers x 1,100 decode steps from an empty cache
    (past one 1,024-token chunk), every step of every layer against the C
    oracle's per-token loop over rows 0 .. t, then every cache byte."""
    import torch

    from insitu_amd import _lib
    from insitu_amd.runtime import ptr
    from insitu_amd.workload import Workload

    L, S = 2, 1100
    wire = [Workload(seed=1000 + l).steps(S) for l in range(L)]
    caches = [_cache(ctx, S) for _ in range(L)]
    dev = [tuple(ctx.to_device(x[0], torch.int32) for x in w) for w in wire]
    outs = torch.empty((L, S, 32, 64), dtype=torch.int32, device=ctx.torch_device)
    for t in range(S):
        for l in range(L):
            qd, kd, vd = dev[l]
            _lib.check(ctx.lib.insitu_step(caches[l].handle, ptr(qd[t]), ptr(kd[t]), ptr(vd[t]),
                                           ptr(outs[l, t]), _lib.MODES[mode], None))
    got = outs.cpu().numpy()
    sg = signs_from_seed(64, 0, 1)
    for l in range(L):
        q, k, v = (np.asarray(x[0], dtype=np.int64) for x in wire[l])
        qr = rotate(q.reshape(-1, 64), sg).reshape(S, 32, 64)
        kr = rotate(k.reshape(-1, 64), sg).reshape(S, 8, 64)
        vr = rotate(v.reshape(-1, 64), sg).reshape(S, 8, 64)
        heads = [encode(kr[:, h], vr[:, h], FMT) for h in range(8)]
        if mode == "online":
            want = native.decode_steps(qr, heads, FMT)
        else:   # two-pass: spot steps (the C checker walks the online order)
            want = got[l].copy()
            for t in (0, 1, 511, 1023, 1024, S - 1):
                want[t] = np.concatenate([native.attend_two_pass(qr[t, 4 * h:4 * h + 4],
                                                                 heads[h].select(slice(0, t + 1)), FMT)[0]
                                          for h in range(8)])
        bad = np.nonzero((got[l] != want).reshape(S, -1).any(axis=1))[0]
        assert bad.size == 0, f"layer {l}: steps {bad[:10].tolist()} differ"
        rows = np.stack([pack(hd, FMT) for hd in heads], axis=1)
        np.testing.assert_array_equal(caches[l].buf, rows, err_msg=f"layer {l} cache bytes")


# -- the chunked kernels: their own edge cases --------------------------------------

def _host_reference(k, v, q, f=FMT, two_pass=False):
    T = k.shape[0]
    host = Cache(8, T, f)
    host.append_rotated(k, v)
    fn = native.attend_two_pass if two_pass else native.attend_online
    outs, sts = [], []
    for h in range(8):
        o, s = fn(q[4 * h:4 * h + 4], host.view(h), f)
        outs.append(o)
        sts.append(s)
    return np.concatenate(outs), sts


def test_chunked_equals_serial_and_counts_the_same_events(ctx):
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(21)
    T = 2600
    k, v = _random_cache_inputs(rng, T)
    c = _cache(ctx, T)
    c.append_rotated(k, v)
    q = rng.integers(-(1 << 22), 1 << 22, size=(32, 64))
    a = CompressedAttention(c)
    o1, s1 = a.attend(q[None], "online")
    o2, s2 = a.attend(q[None], "serial")
    np.testing.assert_array_equal(o1.cpu().numpy(), o2.cpu().numpy())
    want, sts = _host_reference(k, v, q)
    np.testing.assert_array_equal(o1.cpu().numpy()[0], want)
    for st in (s1, s2):
        assert st.rescale_events == sum(s.rescale_events for s in sts)
        assert st.score_overflows == sum(s.score_overflows for s in sts)
        assert st.max_abs_score == max(s.max_abs_score for s in sts)
        assert st.max_abs_acc == max(s.max_abs_acc for s in sts)
        assert st.n_tokens == T and st.acc_overflows == 0
    assert s1.serial_fallbacks == 0


def test_rising_scores_exhaust_the_run_pool_and_fall_back_exactly(ctx):
    """Every token a new maximum: thousands of rescale events; the run pool overflows and
    the affected heads are recomputed serially (still bit-exact)."""
    from insitu_amd.attention import CompressedAttention
    T = 1500
    rng = np.random.default_rng(22)
    base = rng.integers(-(1 << 20), 1 << 20, size=(1, 8, 64))
    grow = (np.arange(1, T + 1)[:, None, None] * 2000)
    k = np.clip(base + grow * np.sign(base), -(1 << 23), (1 << 23) - 1)
    v = rng.integers(-(1 << 20), 1 << 20, size=(T, 8, 64))
    c = _cache(ctx, T)
    c.append_rotated(k, v)
    # q aligned with the key direction so scores grow with the norm
    qv = np.sign(base[0]).repeat(4, axis=0) * (1 << 18)
    out, st = CompressedAttention(c).attend(qv[None], "online")
    want, sts = _host_reference(k, v, qv)
    np.testing.assert_array_equal(out.cpu().numpy()[0], want)
    assert st.rescale_events == sum(s.rescale_events for s in sts) > 500


def test_out_of_range_query_falls_back_exactly(ctx):
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(23)
    T = 700
    k, v = _random_cache_inputs(rng, T)
    c = _cache(ctx, T)
    c.append_rotated(k, v)
    q = rng.integers(-(1 << 22), 1 << 22, size=(32, 64))
    q[4:8] = rng.integers(1 << 29, 1 << 30, size=(4, 64)) * rng.choice([-1, 1], size=(4, 64))
    out, st = CompressedAttention(c).attend(q[None], "online")
    want, _ = _host_reference(k, v, q)
    np.testing.assert_array_equal(out.cpu().numpy()[0], want)
    assert st.serial_fallbacks == 4 and st.range_errors > 0


@pytest.mark.parametrize("mode", ["online", "two_pass"])
def test_full_c2_context_against_native_oracle(ctx, mode):
    """ctx 32,768 (BASELINE config 2 size) on the workload's own distribution."""
    from insitu_amd.attention import CompressedAttention
    from insitu_amd.rotate import Rotation
    from insitu_amd.workload import Workload
    T = 32768
    q, k, v = Workload(seed=0).steps(T)
    sg = signs_from_seed(64, 0, 1)
    kr, vr = rotate(k[0], sg), rotate(v[0], sg)
    qr = rotate(q[0, -1], sg)
    c = _cache(ctx, T)
    c.append_rotated(kr, vr)
    out, st = CompressedAttention(c).attend(qr[None], mode)
    want, sts = _host_reference(kr, vr, qr, two_pass=(mode == "two_pass"))
    np.testing.assert_array_equal(out.cpu().numpy()[0], want)
    assert st.serial_fallbacks == 0
    assert st.rescale_events == sum(s.rescale_events for s in sts)


def test_ragged_batch_multi_chunk(ctx):
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(24)
    lens = [1500, 1, 513, 512, 0, 2049]
    c = _cache(ctx, 2100, batch=len(lens))
    data = []
    for b, T in enumerate(lens):
        k, v = _random_cache_inputs(rng, max(T, 1))
        if T:
            c.append_rotated(k[:T], v[:T], seq=b)
        data.append((k[:T], v[:T]))
    q = rng.integers(-(1 << 22), 1 << 22, size=(len(lens), 32, 64))
    for mode in ("online", "two_pass"):
        out, _ = CompressedAttention(c).attend(q, mode)
        out = out.cpu().numpy()
        for b, (k, v) in enumerate(data):
            if k.shape[0] == 0:
                assert not out[b].any()
                continue
            want, _ = _host_reference(k, v, q[b], two_pass=(mode == "two_pass"))
            np.testing.assert_array_equal(out[b], want, err_msg=f"{mode} seq {b}")


@pytest.mark.parametrize("mode", ["online", "two_pass"])
def test_many_chains_merge_their_statistics(ctx, mode):
    """With more than 32 (sequence, KV head) chains the attend merges each chain's four
    heads' statistics in LDS and sends them once. Here 48 ragged chains, and one KV group
    whose queries are out of range goes to the serial path, which merges its own: every
    total equals the oracle's over all chains."""
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(25)
    lens = [1500, 1, 513, 2049, 700, 1024]
    c = _cache(ctx, 2100, batch=len(lens))
    data = []
    for b, T in enumerate(lens):
        k, v = _random_cache_inputs(rng, T)
        c.append_rotated(k, v, seq=b)
        data.append((k, v))
    q = rng.integers(-(1 << 22), 1 << 22, size=(len(lens), 32, 64))
    q[3, 4:8] = rng.integers(1 << 29, 1 << 30, size=(4, 64)) * rng.choice([-1, 1], size=(4, 64))
    out, st = CompressedAttention(c).attend(q, mode)
    out = out.cpu().numpy()
    sts = []
    for b, (k, v) in enumerate(data):
        want, s = _host_reference(k, v, q[b], two_pass=(mode == "two_pass"))
        np.testing.assert_array_equal(out[b], want, err_msg=f"{mode} seq {b}")
        sts += s
    if mode == "online":
        assert st.serial_fallbacks == 4
    assert st.range_errors > 0
    assert st.n_tokens == max(lens)
    assert st.rescale_events == sum(s.rescale_events for s in sts)
    assert st.rescale_events > 0 or mode == "two_pass"      # two-pass never rescales
    assert st.max_abs_acc == max(s.max_abs_acc for s in sts)
    assert st.acc_overflows == sum(s.acc_overflows for s in sts)
    assert st.max_abs_score == max(s.max_abs_score for s in sts)
    assert st.score_overflows == sum(s.score_overflows for s in sts)


def _host_reference_kv(k, v, q, n_kv, two_pass=False):
    """Per KV group oracle outputs for any number of KV heads (4 query heads each)."""
    T = k.shape[0]
    host = Cache(n_kv, T, FMT)
    host.append_rotated(k, v)
    fn = native.attend_two_pass if two_pass else native.attend_online
    outs, sts = [], []
    for h in range(n_kv):
        o, s = fn(q[4 * h:4 * h + 4], host.view(h), FMT)
        outs.append(o)
        sts.append(s)
    return np.concatenate(outs), sts


@pytest.mark.parametrize("n_kv,lens", [
    (2, [5000, 3100, 4097]),            # 6 (sequence, KV head) chains
    (1, [9000, 2500, 1, 7000, 4200]),   # 5 chains
    (3, [20000]),                       # 3 chains, 20 chunks each
])
def test_chains_that_straddle_xcds(ctx, n_kv, lens):
    """Workgroups are numbered chunk-major and dispatched round-robin over the 8
    XCDs, so with a chain count that is not a multiple of 8 the chunks of one
    chain run on different XCDs: the look-back words, run sums, headers and
    completion counter are then exchanged across XCD L2s."""
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(sum(lens) + n_kv)
    c = _cache(ctx, max(lens), batch=len(lens), n_kv=n_kv, n_q=4 * n_kv)
    data = []
    for b, T in enumerate(lens):
        k, v = _random_cache_inputs(rng, T, n_kv=n_kv)
        c.append_rotated(k, v, seq=b)
        data.append((k, v))
    q = rng.integers(-(1 << 22), 1 << 22, size=(len(lens), 4 * n_kv, 64))
    for mode in ("online", "two_pass"):
        for rep in range(2):
            out, st = CompressedAttention(c).attend(q, mode)
            out = out.cpu().numpy()
            events = 0
            for b, (k, v) in enumerate(data):
                want, sts = _host_reference_kv(k, v, q[b], n_kv, two_pass=(mode == "two_pass"))
                np.testing.assert_array_equal(out[b], want, err_msg=f"{mode} rep {rep} seq {b}")
                events += sum(s.rescale_events for s in sts)
            assert st.serial_fallbacks == 0
            assert st.rescale_events == events


def test_a_later_chunk_replays_from_chunk_zeros_published_state(ctx):
    """Chunk 0 replays its own runs and keeps the result in registers when it is the
    chain's last workgroup. Here the last chunk is much slower (1,024 tied top scores:
    one event, then a candidate per token), so it replays instead and takes chunk 0's
    state from memory once chunk 0's header is up."""
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(31)
    T = 3 * 1024
    qg = rng.integers(-(1 << 22), 1 << 22, size=(8, 64))
    q = np.repeat(qg, 4, axis=0)
    k, v = _random_cache_inputs(rng, T, scale=1 << 17)
    k[2 * 1024:] = (np.sign(qg) * (1 << 22))[None]
    c = _cache(ctx, T)
    c.append_rotated(k, v)
    want, sts = _host_reference(k, v, q)
    for mode in ("online", "two_pass"):
        if mode == "two_pass":
            want, sts = _host_reference(k, v, q, two_pass=True)
        for rep in range(3):
            out, st = CompressedAttention(c).attend(q[None], mode)
            np.testing.assert_array_equal(out.cpu().numpy()[0], want, err_msg=f"{mode} rep {rep}")
            assert st.serial_fallbacks == 0
            assert st.rescale_events == sum(s.rescale_events for s in sts)


@pytest.mark.parametrize("pin", ["chunked", "scan"])
def test_short_contexts_in_a_large_cache(ctx, pin):
    """A cache sized for 131,072 tokens holding 1, 100 and then 1,500 rows: the grid
    follows the longest sequence, not the capacity, and every length is exact (the
    fused step included, whose grid covers the new row's chunk)."""
    from insitu_amd import ModelConfig, QuantConfig
    from insitu_amd.attention import CompressedAttention
    from insitu_amd.block import AttentionBlock
    rng = np.random.default_rng(61)
    blk = AttentionBlock(ModelConfig.llama32_1b(), QuantConfig(key_bits=4, value_bits=2),
                         capacity=131072, softmax="online", ctx=ctx)
    blk.cache.pin_kernel(pin)
    host = Cache(8, 1600, FMT)
    sg = signs_from_seed(64, 0, 1)
    done = 0
    for n in (1, 99, 1400):
        k, v = _random_cache_inputs(rng, n)
        blk.cache.append_rotated(k, v)
        host.append_rotated(k, v)
        done += n
        q = rng.integers(-(1 << 22), 1 << 22, size=(32, 64))
        out, st = CompressedAttention(blk.cache).attend(q[None], "online")
        want = np.concatenate([native.attend_online(q[4 * h:4 * h + 4], host.view(h), FMT)[0]
                               for h in range(8)])
        np.testing.assert_array_equal(out.cpu().numpy()[0], want, err_msg=f"ctx {done}")
        assert st.serial_fallbacks == 0 and st.n_tokens == done
        qw, kw, vw = (rng.integers(-(1 << 22), 1 << 22, size=(1, h, 64)) for h in (32, 8, 8))
        got = blk.step(qw, kw, vw).cpu().numpy()[0]
        host.append_rotated(rotate(kw[0], sg)[None], rotate(vw[0], sg)[None])
        done += 1
        qr = rotate(qw[0], sg)
        want = np.concatenate([native.attend_online(qr[4 * h:4 * h + 4], host.view(h), FMT)[0]
                               for h in range(8)])
        np.testing.assert_array_equal(got, want.reshape(-1), err_msg=f"step at ctx {done}")


def test_repeated_calls_reuse_the_counters(ctx):
    """The chunk-completion and run-pool counters are reset by each call's last workgroup."""
    from insitu_amd.attention import CompressedAttention
    rng = np.random.default_rng(25)
    T = 1300
    k, v = _random_cache_inputs(rng, T)
    c = _cache(ctx, T + 10)
    c.append_rotated(k[:1000], v[:1000])
    a = CompressedAttention(c)
    q = rng.integers(-(1 << 22), 1 << 22, size=(32, 64))
    first, _ = a.attend(q[None], "online")
    for _ in range(5):
        again, _ = a.attend(q[None], "online")
        np.testing.assert_array_equal(again.cpu().numpy(), first.cpu().numpy())
    c.append_rotated(k[1000:], v[1000:])
    out, _ = a.attend(q[None], "online")
    want, _ = _host_reference(k, v, q)
    np.testing.assert_array_equal(out.cpu().numpy()[0], want)


# -- the fused decode step (one write kernel, then the attend) at multi-chunk contexts --

@pytest.mark.parametrize("mode", ["online", "two_pass", "serial"])
@pytest.mark.parametrize("d,kb,vb", [(64, 4, 2), (128, 3, 3)])
def test_fused_step_ragged_batch_multi_chunk(ctx, mode, d, kb, vb):
    """insitu_step over a ragged batch whose caches span several chunks: every
    sequence's output against the oracle's attend on the host-rotated query, and
    the rows the step appended byte for byte (kernel.py:271-345)."""
    from insitu_amd import ModelConfig, QuantConfig
    from insitu_amd.block import AttentionBlock
    rng = np.random.default_rng(31 + d)
    lens, steps, batch = [2500, 1100], 2, 2
    model = ModelConfig.llama32_1b() if d == 64 else ModelConfig(
        hidden_size=4096, num_heads=32, num_kv_heads=8, head_dim=128)
    f = Format(d=d, key_bits=kb, value_bits=vb)
    blk = AttentionBlock(model, QuantConfig(key_bits=kb, value_bits=vb),
                         capacity=max(lens) + steps, batch=batch, softmax=mode, ctx=ctx)
    sg = signs_from_seed(d, 0, 1)
    hosts = []
    for b, T in enumerate(lens):
        k, v = _random_cache_inputs(rng, T, d=d)
        blk.cache.append_rotated(k, v, seq=b)
        h = Cache(8, T + steps, f)
        h.append_rotated(k, v)
        hosts.append(h)
    fn = native.attend_two_pass if mode == "two_pass" else native.attend_online
    for t in range(steps):
        qw = rng.integers(-(1 << 23), 1 << 23, size=(batch, 32, d))
        kw = rng.integers(-(1 << 23), 1 << 23, size=(batch, 8, d))
        vw = rng.integers(-(1 << 23), 1 << 23, size=(batch, 8, d))
        out = blk.step(qw, kw, vw).cpu().numpy().reshape(batch, 32, d)
        for b in range(batch):
            qr, kr, vr = rotate(qw[b], sg), rotate(kw[b], sg), rotate(vw[b], sg)
            hosts[b].append_rotated(kr[None], vr[None])
            want = np.concatenate([fn(qr[4 * g:4 * g + 4], hosts[b].view(g), f)[0]
                                   for g in range(8)])
            np.testing.assert_array_equal(out[b], want, err_msg=f"step {t} seq {b}")
        assert blk.last_stats.serial_fallbacks == 0 and blk.last_stats.range_errors == 0
    for b, T in enumerate(lens):
        for g in (0, 7):
            np.testing.assert_array_equal(blk.cache.read_rows(g, T, steps, seq=b),
                                          hosts[b].buf[T:T + steps, g])


def test_fused_step_over_a_flat_softmax(ctx):
    """insitu_step with small queries over the workload's rows: nearly every token of every
    chunk is a candidate, so the fused step's run-sum walk takes its long paths (event-free
    groups, prefix tracking of runs whose bound passes 2^24) that peaked queries skip."""
    from insitu_amd import ModelConfig, QuantConfig
    from insitu_amd.block import AttentionBlock
    from insitu_amd.workload import Workload
    T, steps = 3000, 3
    q_w, k_w, v_w = Workload(seed=7).steps(T + steps)
    sg = signs_from_seed(64, 0, 1)
    blk = AttentionBlock(ModelConfig.llama32_1b(), QuantConfig(key_bits=4, value_bits=2),
                         capacity=T + steps, ctx=ctx)
    kr = rotate(k_w[0, :T].astype(np.int64), sg)
    vr = rotate(v_w[0, :T].astype(np.int64), sg)
    blk.cache.append_rotated(kr, vr)
    host = Cache(8, T + steps, FMT)
    host.append_rotated(kr, vr)
    rng = np.random.default_rng(8)
    for t in range(steps):
        qw = rng.integers(-(1 << 9), 1 << 9, size=(1, 32, 64))
        kw, vw = k_w[:, T + t], v_w[:, T + t]
        out = blk.step(qw, kw, vw).cpu().numpy().reshape(32, 64)
        host.append_rotated(rotate(kw[0].astype(np.int64), sg)[None], rotate(vw[0].astype(np.int64), sg)[None])
        qr = rotate(qw[0], sg)
        want, sts = [], []
        for g in range(8):
            o, st_g = native.attend_online(qr[4 * g:4 * g + 4], host.view(g), FMT)
            want.append(o)
            sts.append(st_g)
        np.testing.assert_array_equal(out, np.concatenate(want), err_msg=f"step {t}")
        st = blk.last_stats
        assert st.serial_fallbacks == 0
        assert st.rescale_events == sum(x.rescale_events for x in sts)
        assert st.max_abs_acc == max(x.max_abs_acc for x in sts)


@pytest.mark.parametrize("mode", ["online", "serial"])
def test_fused_step_counts_rotated_queries_beyond_the_seam_range(ctx, mode):
    """A wire query of 2^30 on one channel rotates to +-2^27 on every channel,
    beyond what the 24-bit seam can produce: each such value is one range
    error (once per call, whichever attend runs), and the output stays exact,
    since ||q||_1 * max|c| is still below 2^51."""
    from insitu_amd import ModelConfig, QuantConfig
    from insitu_amd.block import AttentionBlock
    rng = np.random.default_rng(41)
    T = 1500
    blk = AttentionBlock(ModelConfig.llama32_1b(), QuantConfig(key_bits=4, value_bits=2),
                         capacity=T + 1, softmax=mode, ctx=ctx)
    k, v = _random_cache_inputs(rng, T)
    blk.cache.append_rotated(k, v)
    host = Cache(8, T + 1, FMT)
    host.append_rotated(k, v)
    qw = rng.integers(-(1 << 22), 1 << 22, size=(1, 32, 64))
    qw[0, 8:12] = 0
    qw[0, 8:12, 0] = 1 << 30
    kw = rng.integers(-(1 << 22), 1 << 22, size=(1, 8, 64))
    vw = rng.integers(-(1 << 22), 1 << 22, size=(1, 8, 64))
    out = blk.step(qw, kw, vw).cpu().numpy().reshape(32, 64)
    sg = signs_from_seed(64, 0, 1)
    qr = rotate(qw[0], sg)
    assert np.all(np.abs(qr[8:12]) == 1 << 27)
    host.append_rotated(rotate(kw[0], sg)[None], rotate(vw[0], sg)[None])
    want = np.concatenate([native.attend_online(qr[4 * g:4 * g + 4], host.view(g), FMT)[0]
                           for g in range(8)])
    np.testing.assert_array_equal(out, want)
    st = blk.last_stats
    assert st.range_errors == 4 * 64 and st.serial_fallbacks == 0


def test_attend_timing_hook_counts_every_attend(ctx):
    """insitu_ctx_timing: one event pair per attend, in both the standalone attend
    and the fused step; the summed kernel time is positive and read once."""
    import ctypes

    from insitu_amd import ModelConfig, QuantConfig, _lib
    from insitu_amd.attention import CompressedAttention
    from insitu_amd.block import AttentionBlock
    rng = np.random.default_rng(5)
    blk = AttentionBlock(ModelConfig.llama32_1b(), QuantConfig(key_bits=4, value_bits=2),
                         capacity=2100, ctx=ctx)
    k, v = _random_cache_inputs(rng, 2048)
    blk.cache.append_rotated(k, v)
    lib = ctx.lib
    ms, n = ctypes.c_double(), ctypes.c_int64()
    _lib.check(lib.insitu_ctx_timing(ctx.handle, 1))
    try:
        q = rng.integers(-(1 << 22), 1 << 22, size=(1, 32, 64))
        CompressedAttention(blk.cache).attend(q, "online", stats=False)
        CompressedAttention(blk.cache).attend(q, "two_pass", stats=False)
        for _ in range(3):
            blk.step(q, k[:1], v[:1], stats=False)
        _lib.check(lib.insitu_ctx_timing_read(ctx.handle, ctypes.byref(ms), ctypes.byref(n)))
        assert n.value == 5 and ms.value > 0.0
        _lib.check(lib.insitu_ctx_timing_read(ctx.handle, ctypes.byref(ms), ctypes.byref(n)))
        assert n.value == 0 and ms.value == 0.0
    finally:
        _lib.check(lib.insitu_ctx_timing(ctx.handle, 0))


# -- prefill: every query of a prompt at once (attention.py:517-871) ------------------

@pytest.mark.parametrize("kb,vb", [(4, 2), (3, 2), (2, 3)])
@pytest.mark.parametrize("mode", ["online", "two_pass", "serial"])
def test_prefill_is_the_token_loop(ctx, kb, vb, mode):
    """attend_online_batch / attend_causal_batch are the per-query loop, bit for bit
    (the reference's check_online_batch_is_bit_identical and
    check_causal_batch_is_bit_identical): query t attends rows 0 .. t."""
    from insitu_amd.attention import CompressedAttention
    f = Format(key_bits=kb, value_bits=vb)
    T = 53
    rng = np.random.default_rng(kb * 10 + vb)
    k, v = _random_cache_inputs(rng, T)
    c = _cache(ctx, T, kb=kb, vb=vb)
    c.append_rotated(k, v)
    q = rng.integers(-(1 << 22), 1 << 22, size=(T, 32, 64))
    out, st = CompressedAttention(c).attend_prefill(q, 0, mode)
    out = out.cpu().numpy()
    host = Cache(8, T, f)
    host.append_rotated(k, v)
    fn = attend_two_pass if mode == "two_pass" else attend_online
    events = 0
    for t in range(T):
        for h in range(8):
            want, s = fn(q[t, 4 * h:4 * h + 4], host.view(h).select(slice(0, t + 1)), f)
            np.testing.assert_array_equal(out[t, 4 * h:4 * h + 4], want, err_msg=f"query {t} group {h}")
            events += s.rescale_events
    assert st.rescale_events == events
    if mode != "two_pass":
        assert events > 0


@pytest.mark.parametrize("mode", ["online", "two_pass"])
def test_prefill_from_a_base_across_chunks_and_query_batches(ctx, mode):
    """600 queries from row 2,000 of a 2,600-row cache: the queries cross a
    1,024-token chunk boundary and the 256-query launches of the virtual batch;
    every query against the C oracle over rows 0 .. base + i."""
    from insitu_amd.attention import CompressedAttention
    base, n_q = 2000, 600
    T = base + n_q
    rng = np.random.default_rng(5)
    k, v = _random_cache_inputs(rng, T)
    c = _cache(ctx, T)
    c.append_rotated(k, v)
    q = rng.integers(-(1 << 22), 1 << 22, size=(n_q, 32, 64))
    out, _ = CompressedAttention(c).attend_prefill(q, base, mode)
    out = out.cpu().numpy()
    host = Cache(8, T, FMT)
    host.append_rotated(k, v)
    heads = [host.view(h) for h in range(8)]
    if mode == "online":
        want = native.decode_steps(q, heads, FMT, base=base)
        bad = np.nonzero((out != want).reshape(n_q, -1).any(axis=1))[0]
        assert bad.size == 0, f"queries {bad[:10].tolist()} differ"
    else:
        for i in (0, 47, 255, 256, 511, n_q - 1):
            want = np.concatenate([native.attend_two_pass(q[i, 4 * h:4 * h + 4],
                                                          heads[h].select(slice(0, base + i + 1)), FMT)[0]
                                   for h in range(8)])
            np.testing.assert_array_equal(out[i], want, err_msg=f"query {i}")


def test_prefill_group_interface_and_bounds(ctx):
    """The reference-shaped per-group calls, and EBADLEN past the cache's rows."""
    from insitu_amd import _lib
    from insitu_amd.attention import CompressedAttention
    T = 40
    rng = np.random.default_rng(3)
    k, v = _random_cache_inputs(rng, T)
    c = _cache(ctx, T + 10)
    c.append_rotated(k, v)
    host = Cache(8, T, FMT)
    host.append_rotated(k, v)
    a = CompressedAttention(c)
    q = rng.integers(-(1 << 22), 1 << 22, size=(12, 4, 64))
    got, _ = a.attend_online_batch(q, c.view(5), base=T - 12)
    got2, _ = a.attend_causal_batch(q, c.view(5), base=T - 12)
    for i in range(12):
        view = host.view(5).select(slice(0, T - 12 + i + 1))
        np.testing.assert_array_equal(got[i], attend_online(q[i], view, FMT)[0])
        np.testing.assert_array_equal(got2[i], attend_two_pass(q[i], view, FMT)[0])
    with pytest.raises(_lib.InsituError, match="EBADLEN"):
        a.attend_prefill(np.zeros((12, 32, 64), dtype=np.int32), T - 11, "online")


@pytest.mark.parametrize("softmax", ["online", "two_pass"])
def test_block_prefill_equals_the_decode_loop(ctx, softmax):
    """kernel.py:316-341: a prompt through prefill gives the same outputs and the
    same cache bytes as the same tokens one decode step at a time, also when
    the prompt follows earlier tokens (base > 0)."""
    from insitu_amd import ModelConfig, QuantConfig
    from insitu_amd.block import AttentionBlock
    from insitu_amd.workload import Workload
    q, k, v = Workload(seed=7).steps(330)
    q, k, v = q[0], k[0], v[0]
    mk = lambda: AttentionBlock(ModelConfig.llama32_1b(), QuantConfig(key_bits=4, value_bits=2),
                                capacity=330, softmax=softmax, ctx=ctx)
    loop, pre = mk(), mk()
    want = loop.forward_seam(q, k, v, force_token_loop=True)
    got_a = pre.forward_seam(q[:30], k[:30], v[:30])          # a first prompt
    got_b = pre.forward_seam(q[30:], k[30:], v[30:])          # continues at base 30
    np.testing.assert_array_equal(np.concatenate([got_a, got_b]), want)
    np.testing.assert_array_equal(pre.cache.buf, loop.cache.buf)


# -- cache image interop -----------------------------------------------------------

def test_cache_image_round_trip_and_device_diff(ctx, fixture_cache):
    """ddr_layout.py:227-257, CMD_LOAD and experiments/cache_diff.py: the golden
    plane image installed verbatim into a fresh cache reads back as the golden
    rows and attends to the golden output; the device diff of a cache against
    its own rows matches, and a byte planted in the host's copy is named."""
    from insitu_amd.attention import CompressedAttention
    from insitu_amd.interop import DdrLayout, diff_device_cache
    c0, rows = fixture_cache
    c = _cache(ctx, 65)
    lay = DdrLayout.for_cache(c)
    img = lay.image(rows)
    np.testing.assert_array_equal(img, hx.bytes_rows("ddr_image.hex").reshape(-1))
    c.load_image(img)
    c.set_length(65)
    np.testing.assert_array_equal(c.buf, rows)
    np.testing.assert_array_equal(c.image(), img)
    q = hx.lanes("rot_q.hex", 24, 64)
    out, _ = CompressedAttention(c).attend(q[None], "online")
    np.testing.assert_array_equal(out.cpu().numpy().reshape(-1), hx.lanes("out.online.hex", 24, 2048)[0])
    assert diff_device_cache(c, rows).match
    host = rows.copy()
    host[17, 6, 49] ^= 4
    rep = diff_device_cache(c0, host)
    assert [(r.head, r.token, r.fields) for r in rep.rows] == [(6, 17, ["norms"])]
