"""The oracle against what the mathematics fixes, where the fixtures leave room.

Each check is chosen so a plausible slip (a dropped term, a wrong rounding
side, a transposed operand) fails it.
"""

import math

import numpy as np
import pytest

from oracle import native
from oracle.attention import ExpLut, attend_online, attend_two_pass, reciprocal, scores
from oracle.codebook import gaussian
from oracle.fixed import Q, fwht, inv_sqrt_q15, rshift, sqrt_shift
from oracle.quantize import (CompressedKV, Format, decode_plane, isqrt, pack, pack_codes, unpack,
                             unpack_codes)
from oracle.rotate import inverse_rotate, matrix, rotate, signs_from_seed

FMT = Format()


def test_rshift_rounding_tie_tables():
    # value / 2 for -3..3: floor, half-up (towards +inf on ties), half-even.
    x = np.arange(-3, 4)
    np.testing.assert_array_equal(rshift(x, 1, "floor"), [-2, -1, -1, 0, 0, 1, 1])
    np.testing.assert_array_equal(rshift(x, 1, "up"), [-1, -1, 0, 0, 1, 1, 2])
    np.testing.assert_array_equal(rshift(x, 1, "even"), [-2, -1, 0, 0, 0, 1, 2])
    np.testing.assert_array_equal(rshift(np.array([6, 10, 14, 2]), 2, "even"), [2, 2, 4, 0])
    np.testing.assert_array_equal(rshift(x, 0), x)
    np.testing.assert_array_equal(rshift(np.array([5, 7]), np.array([0, 1]), "even"), [5, 4])
    with pytest.raises(ValueError):
        rshift(x, -1)


def test_q_clamp_and_from_float():
    q = Q(24, 16)
    assert (q.lo, q.hi) == (-(1 << 23), (1 << 23) - 1)
    np.testing.assert_array_equal(q.from_float([0.5 / 65536, 1.5 / 65536, 1e9, -1e9]),
                                  [0, 2, q.hi, q.lo])


def test_fwht_equals_the_dense_sylvester_hadamard():
    rng = np.random.default_rng(1)
    for n in (2, 8, 64, 128):
        h = np.array([[1]])
        while h.shape[0] < n:
            h = np.block([[h, h], [h, -h]])
        x = rng.integers(-(1 << 20), 1 << 20, size=(5, n))
        np.testing.assert_array_equal(fwht(x), x @ h.T)


def test_sqrt_shift_and_q15():
    assert [sqrt_shift(n) for n in (1, 4, 16, 64, 256, 32, 128, 12)] == [0, 1, 2, 3, 4, None, None, None]
    assert inv_sqrt_q15(128) == 2896 and inv_sqrt_q15(32) == 5793


def test_rotation_matches_the_dense_matrix_within_the_floor():
    rng = np.random.default_rng(2)
    for d in (64, 128):
        s = signs_from_seed(d, 7, 1)
        x = rng.integers(-(1 << 20), 1 << 20, size=(16, d))
        exact = x @ matrix(s).T
        got = rotate(x, s)
        err = exact - got
        # d=64: the scale is an exact >>3, so only the floor is lost: 0 <= err < 1.
        # d=128: 2896/2^15 differs from 1/sqrt(128) by `rel`, applied to the
        # unnormalised transform (|exact| * sqrt(128)), then floored.
        rel = abs(2896 / 32768 - 1 / math.sqrt(128)) if d == 128 else 0.0
        slack = np.abs(exact) * math.sqrt(d) * rel + 1e-6
        assert np.all(err >= -slack) and np.all(err < 1 + slack), d


def test_rotation_seed_is_numpy_pcg64_and_d128_has_two_words():
    s = signs_from_seed(128, 0, 1)
    rng = np.random.Generator(np.random.PCG64(0))
    np.testing.assert_array_equal(s, rng.integers(0, 2, size=(1, 128)) * 2 - 1)
    np.testing.assert_array_equal(signs_from_seed(64, 0, 1)[0], s[0, :64])


def test_inverse_rotation_round_trip_loses_only_truncation():
    rng = np.random.default_rng(3)
    s = signs_from_seed(64, 0, 2)
    x = rng.integers(-(1 << 22), 1 << 22, size=(8, 64))
    back = inverse_rotate(rotate(x, s), s)
    # Four floor stages (two rounds each way), each off by < 1 per channel,
    # i.e. < sqrt(d) in norm; the orthonormal stages carry it unchanged.
    assert np.all(np.linalg.norm(back - x, axis=1) < 4 * np.sqrt(64))


def test_isqrt_invariant():
    rng = np.random.default_rng(4)
    a = np.concatenate([np.arange(0, 2000), rng.integers(0, 1 << 58, 5000),
                        [(1 << 52) - 1, 1 << 52, (1 << 58) - 1]])
    r = isqrt(a)
    assert np.all(r * r <= a) and np.all((r + 1) * (r + 1) > a)
    for v in (0, 1, 2, 3, 4, 99, 10 ** 12 + 7):
        assert int(isqrt(np.array([v]))[0]) == math.isqrt(v)


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 8])
def test_pack_unpack_round_trip_every_width(bits):
    rng = np.random.default_rng(bits)
    for d in (64, 128):
        idx = rng.integers(0, 1 << bits, size=(17, d)).astype(np.uint8)
        buf = pack_codes(idx, bits)
        assert buf.shape == (17, d * bits // 8)
        np.testing.assert_array_equal(unpack_codes(buf, bits, d), idx)
        # LSB-first bitstream: channel c's bit j is stream bit c*bits + j.
        stream = np.unpackbits(buf, axis=1, bitorder="little")
        for c in (0, 1, d - 1):
            for j in range(bits):
                assert np.array_equal(stream[:, c * bits + j], (idx[:, c] >> j) & 1)


def test_row_round_trip_3b3b_d128_and_signed_norms():
    f = Format(d=128, key_bits=3, value_bits=3)
    assert f.row_bytes == 100
    rng = np.random.default_rng(5)
    kv = CompressedKV(rng.integers(0, 8, (9, 128)).astype(np.uint8),
                      np.array([0, 1, -1, 32767, -32768, 5, 6, 7, 8]),
                      rng.integers(0, 8, (9, 128)).astype(np.uint8),
                      np.array([-5, 4, 3, 2, 1, 0, -1, -2, -32768]))
    back = unpack(pack(kv, f), f)
    for a, b in zip((kv.k_idx, kv.k_norm, kv.v_idx, kv.v_norm),
                    (back.k_idx, back.k_norm, back.v_idx, back.v_norm)):
        np.testing.assert_array_equal(a, b)


def test_codebooks_match_published_lloyd_max_and_are_symmetric():
    known = {2: [0.4528, 1.5104], 3: [0.2451, 0.7560, 1.3439, 2.1520]}
    for bits, pos in known.items():
        c, b = gaussian(bits)
        got = c.astype(np.float64)[len(c) // 2:] / (1 << 15)
        np.testing.assert_allclose(got, pos, atol=2e-3)
        np.testing.assert_array_equal(c, -c[::-1])
        np.testing.assert_array_equal(b, (c[:-1] + c[1:]) >> 1)


def test_exp_lut_is_exp_within_one_lsb_and_monotone():
    e = ExpLut(FMT)
    d = np.arange(0, int(e.delta_max) + 10, 37)
    p = e(d)
    want = np.exp(-d / 65536.0) * 32768
    assert np.all(np.abs(p - want) <= 1.0 + want * 4e-3)
    assert np.all(np.diff(p) <= 0) and p[-1] == 0 and e(np.array([0]))[0] == 32768
    with pytest.raises(ValueError):
        e(np.array([-1]))


def test_reciprocal_precision_at_every_context():
    for T in (64, 1024, 20000, 24576, 32768, 131072, 1 << 22):
        l = int(round(T * 32768 * 0.998))
        r, sh = reciprocal(np.array([l]), FMT)
        got = int(r[0]) / 2.0 ** int(sh[0])
        assert abs(got - 32768 / l) / (32768 / l) < 1e-6
        assert (1 << 30) < int(r[0]) <= (1 << 31)
    r, sh = reciprocal(np.array([0, 1]), FMT)
    assert int(r[0]) == 0 and int(r[1]) == 1 << 31 and np.all(sh >= 0)


def _random_kv(rng, T, f=FMT):
    return CompressedKV(rng.integers(0, 1 << f.key_bits, (T, f.d)).astype(np.uint8),
                        rng.integers(300, 1500, T),
                        rng.integers(0, 1 << f.value_bits, (T, f.d)).astype(np.uint8),
                        rng.integers(300, 1500, T))


def test_scores_equal_unbounded_python_integers():
    rng = np.random.default_rng(6)
    kv = _random_kv(rng, 40)
    q = rng.integers(-(1 << 23), 1 << 23, size=(4, 64))
    kc = FMT.codebooks()[0]
    s, _ = scores(q, kv, FMT)
    for h in range(4):
        for t in range(40):
            dot = sum(int(q[h, j]) * int(kc[kv.k_idx[t, j]]) for j in range(64))
            assert s[h, t] == (dot * int(kv.k_norm[t])) >> 24


def test_scores_approximate_the_dense_inner_product():
    # <q, k> with k rebuilt from codes: the only difference is the decode truncation.
    rng = np.random.default_rng(7)
    kv = _random_kv(rng, 30)
    q = rng.integers(-(1 << 18), 1 << 18, size=(4, 64))
    kc = FMT.codebooks()[0]
    k = decode_plane(kv.k_idx, kv.k_norm, kc, FMT)
    dense = (q @ k.T) / 65536.0
    s, _ = scores(q, kv, FMT)
    assert np.all(np.abs(s - dense) <= 1 + np.abs(q).sum(axis=1)[:, None] / 65536.0)


def test_online_equals_a_tiny_brute_force_and_two_pass_has_no_rescale():
    rng = np.random.default_rng(8)
    kv = _random_kv(rng, 6)
    q = rng.integers(-(1 << 22), 1 << 22, size=(2, 64))
    e = ExpLut(FMT)
    s, _ = scores(q, kv, FMT)
    vc = FMT.codebooks()[2]
    for h in range(2):
        m, l, acc = -(1 << 47), 0, [0] * 64
        for t in range(6):
            st = int(s[h, t])
            if st > m:
                f = int(e(np.array([st - m]))[0])
                acc = [(a * f) >> 15 for a in acc]
                l = (l * f) >> 15
                m = st
            p = int(e(np.array([m - st]))[0])
            l += p
            acc = [max(-(1 << 31), min((1 << 31) - 1,
                                       a + ((int(kv.v_norm[t]) * p * int(vc[kv.v_idx[t, j]])) >> 23)))
                   for j, a in enumerate(acc)]
        out, _ = attend_online(q[h:h + 1], kv, FMT)
        r, sh = reciprocal(np.array([l]), FMT)
        want = [(a * int(r[0])) >> int(sh[0]) for a in acc]
        np.testing.assert_array_equal(out[0], want)
    _, st = attend_two_pass(q, kv, FMT)
    assert st.rescale_events == 0


def test_native_oracle_equals_numpy_oracle():
    rng = np.random.default_rng(9)
    for f in (FMT, Format(d=128, key_bits=3, value_bits=3)):
        kv = _random_kv(rng, 300, f)
        q = rng.integers(-(1 << 22), 1 << 22, size=(4, f.d))
        q[1] *= 0      # a zero query: every score zero, uniform attention
        s_np, o_np = scores(q, kv, f)
        s_c, o_c = native.scores(q, kv, f)
        np.testing.assert_array_equal(s_np, s_c)
        assert o_np == o_c
        for a, b in ((attend_online(q, kv, f), native.attend_online(q, kv, f)),
                     (attend_two_pass(q, kv, f), native.attend_two_pass(q, kv, f))):
            np.testing.assert_array_equal(a[0], b[0])
            assert a[1] == b[1]
    d = np.arange(0, 800000, 13)
    np.testing.assert_array_equal(native.exp_lut(d, FMT), ExpLut(FMT)(d))


def test_native_decode_steps_equal_the_per_token_loop_step_by_step():
    """The config-1 checker: step t attends rows 0 .. t, each step as attend_online does."""
    rng = np.random.default_rng(12)
    steps, n_kv = 40, 2
    heads = [_random_kv(rng, steps, FMT) for _ in range(n_kv)]
    q = rng.integers(-(1 << 22), 1 << 22, size=(steps, 4 * n_kv, FMT.d))
    q[5] = 0
    got = native.decode_steps(q, heads, FMT)
    for t in (0, 1, 5, 17, steps - 1):
        for h in range(n_kv):
            want, _ = attend_online(q[t, 4 * h:4 * h + 4], heads[h].select(slice(0, t + 1)), FMT)
            np.testing.assert_array_equal(got[t, 4 * h:4 * h + 4], want, err_msg=f"step {t} head {h}")
    # from a base: query i attends rows 0 .. base + i
    base = 25
    got = native.decode_steps(q[base:], heads, FMT, base=base)
    for i in (0, 3, steps - base - 1):
        for h in range(n_kv):
            want, _ = attend_online(q[base + i, 4 * h:4 * h + 4], heads[h].select(slice(0, base + i + 1)), FMT)
            np.testing.assert_array_equal(got[i, 4 * h:4 * h + 4], want, err_msg=f"base {base} query {i}")
