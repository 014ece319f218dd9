"""The CPU oracle against every golden vector the reference ships (tb/vectors).

These pin the oracle before anything is checked against it. The fixtures are
the reference's own data files (hw/vectors.py:379-814 wrote them), copied
verbatim into tests/golden/tb_vectors.
"""

import numpy as np
import pytest

from oracle import hexio as hx
from oracle.attention import (ExpLut, attend_online, attend_two_pass, finalize, qtab,
                              reciprocal, scores)
from oracle.layout import DdrLayout
from oracle.quantize import Format, encode, encode_plane, norm_wire, pack, unpack
from oracle.rotate import rotate, sign_words, signs_from_seed

FMT = Format()
SIGNS = signs_from_seed(64, 0, 1)


@pytest.fixture(scope="module")
def cache_rows():
    return np.stack([hx.bytes_rows(f"cache_rows_h{h}.hex") for h in range(8)], axis=1)


@pytest.fixture(scope="module")
def rot_q():
    return hx.lanes("rot_q.hex", 24, 64)


def test_manifest_is_the_reference_configuration():
    m = hx.manifest()
    assert (m["head_dim"], m["num_heads"], m["num_kv_heads"]) == (64, 32, 8)
    assert (m["key_bits"], m["value_bits"], m["row_bytes"]) == (4, 2, 52)
    assert m["softmax_golden"] == "out.online.hex"
    assert FMT.row_bytes == m["row_bytes"]
    assert FMT.score_shift == 24 and FMT.acc_shift == m["acc_shift"] == 23


def test_sign_word_seed0():
    assert sign_words(SIGNS) == [int(hx.lines("rot_signs.hex")[0], 16)]
    assert sign_words(SIGNS)[0] == 0x81191FF5899001F8


def test_rotation_random_vectors():
    rin = hx.lanes("rot_random_in.hex", 24, 64)
    assert rin.shape == (1024, 64)
    np.testing.assert_array_equal(rotate(rin, SIGNS), hx.lanes("rot_random_out.hex", 24, 64))


@pytest.mark.parametrize("name", ["q", "k", "v"])
def test_rotation_of_the_wire(name):
    w = hx.lanes(f"wire_{name}.hex", 24, 64)
    np.testing.assert_array_equal(rotate(w, SIGNS), hx.lanes(f"rot_{name}.hex", 24, 64))


def test_codebooks():
    kc, kb, vc, vb = FMT.codebooks()
    np.testing.assert_array_equal(kc, hx.scalars("cb_centroids_key.hex", 20))
    np.testing.assert_array_equal(vc, hx.scalars("cb_centroids_value.hex", 20))
    np.testing.assert_array_equal(kb, hx.scalars("enc_bounds_key.hex", 20))
    np.testing.assert_array_equal(vb, hx.scalars("enc_bounds_value.hex", 20))


def test_encoder_norms_and_codes_including_exact_ties():
    x = hx.lanes("enc_in.hex", 24, 64)
    assert x.shape == (560, 64)       # 16 real + 512 random + 32 constructed ties
    _, kb, _, vb = FMT.codebooks()
    n = norm_wire(x, FMT)
    np.testing.assert_array_equal(n, hx.scalars("enc_norm.hex", 16))
    np.testing.assert_array_equal(encode_plane(x, kb, n, FMT),
                                  hx.lanes("enc_idx_key.hex", 8, 64, signed=False))
    np.testing.assert_array_equal(encode_plane(x, vb, n, FMT),
                                  hx.lanes("enc_idx_value.hex", 8, 64, signed=False))


def test_the_appended_row_is_kv_rows(cache_rows):
    rk, rv = hx.lanes("rot_k.hex", 24, 64), hx.lanes("rot_v.hex", 24, 64)
    rows = pack(encode(rk, rv, FMT), FMT)
    np.testing.assert_array_equal(rows, hx.bytes_rows("kv_rows.hex"))
    np.testing.assert_array_equal(cache_rows[-1], rows)
    assert cache_rows.shape == (65, 8, 52)


def test_pack_unpack_round_trip_on_the_cache(cache_rows):
    kv = unpack(cache_rows, FMT)
    np.testing.assert_array_equal(pack(kv, FMT), cache_rows)


def test_ddr_image_and_map(cache_rows):
    lay = DdrLayout.for_format(FMT, 8, 65)
    assert lay.describe() == hx.manifest()["ddr"]
    img = lay.image(cache_rows)
    np.testing.assert_array_equal(img, hx.bytes_rows("ddr_image.hex").reshape(-1))
    for h in range(8):
        for t in (0, 31, 64):
            np.testing.assert_array_equal(lay.row_at(img, h, t), cache_rows[t, h])


def test_qtab(rot_q):
    kc = FMT.codebooks()[0]
    np.testing.assert_array_equal(qtab(rot_q, kc).reshape(32, -1),
                                  hx.lanes("qtab_table.hex", 43, 64 * 16))


def test_scores(cache_rows, rot_q):
    got = np.concatenate([scores(rot_q[4 * h:4 * h + 4], unpack(cache_rows[:, h], FMT), FMT)[0]
                          for h in range(8)])
    np.testing.assert_array_equal(got, hx.lanes("scores.hex", 48, 65))


def test_signed_norm_edge_rows(rot_q):
    rows = hx.bytes_rows("score_edge_rows.hex")
    kv = unpack(rows, FMT)
    assert list(kv.k_norm) == [0, 1, 32767, -32768, -1]
    s, _ = scores(rot_q[0], kv, FMT)
    np.testing.assert_array_equal(s, hx.scalars("score_edge_gold.hex", 48))


def test_exp_lut_table_and_every_reachable_output():
    e = ExpLut(FMT)
    np.testing.assert_array_equal(e.table, hx.scalars("exp_table.hex", 16, signed=False))
    m = hx.manifest()
    assert int(e.log2e) == m["exp_log2e"] and int(e.delta_max) == m["exp_delta_max"]
    d = hx.scalars("exp_in.hex", 48)
    want = hx.scalars("exp_out.hex", 16, signed=False)
    np.testing.assert_array_equal(e(d), want)
    np.testing.assert_array_equal(e.two_step(d), want)


def test_online_softmax_per_token_state(cache_rows, rot_q):
    kv0 = unpack(cache_rows[:, 0], FMT)
    for prefix, q in (("sm", rot_q[:4]), ("sm2", hx.lanes("sm2_q.hex", 24, 64))):
        steps = []
        attend_online(q, kv0, FMT, on_step=lambda t, **kw: steps.append(kw))
        assert len(steps) == 65
        for name, bits, signed in (("s", 48, True), ("m", 48, True), ("p", 16, False),
                                   ("l", 48, True), ("factor", 16, False)):
            got = np.stack([st[name] if st[name] is not None else np.full(4, 32768)
                            for st in steps])
            np.testing.assert_array_equal(got, hx.lanes(f"{prefix}_{name}.hex", bits, 4, signed),
                                          err_msg=f"{prefix}_{name}")
        grew = [int(x, 16) for x in hx.lines(f"{prefix}_grew.hex")]
        assert grew == [sum(int(v) << i for i, v in enumerate(st["grew"])) for st in steps]
        acc = hx.lanes(f"{prefix}_acc.hex", 32, 64).reshape(65, 4, 64)
        np.testing.assert_array_equal(np.stack([st["acc"] for st in steps]), acc)


def test_stress_query_has_many_distinct_factors():
    f = hx.lanes("sm2_factor.hex", 16, 4, signed=False)
    g = np.array([[(int(x, 16) >> i) & 1 for i in range(4)] for x in hx.lines("sm2_grew.hex")])
    assert len(set(f[g.astype(bool)].tolist())) >= 8


def test_end_to_end_online_and_two_pass(cache_rows, rot_q):
    on, tp = [], []
    for h in range(8):
        kv = unpack(cache_rows[:, h], FMT)
        on.append(attend_online(rot_q[4 * h:4 * h + 4], kv, FMT)[0])
        tp.append(attend_two_pass(rot_q[4 * h:4 * h + 4], kv, FMT)[0])
    on = np.concatenate(on).reshape(-1)
    tp = np.concatenate(tp).reshape(-1)
    np.testing.assert_array_equal(on, hx.lanes("out.online.hex", 24, 2048)[0])
    np.testing.assert_array_equal(tp, hx.lanes("out.hex", 24, 2048)[0])
    assert not np.array_equal(on, tp)       # the two softmaxes really differ


def test_finalize_goldens():
    fa = hx.lanes("fin_acc.hex", 32, 64)
    fl = hx.scalars("fin_l.hex", 48)
    r, sh = reciprocal(fl, FMT)
    np.testing.assert_array_equal(r, hx.scalars("fin_recip.hex", 32, signed=False))
    np.testing.assert_array_equal(sh, hx.scalars("fin_shift.hex", 8, signed=False))
    np.testing.assert_array_equal(finalize(fa, fl, FMT), hx.lanes("fin_out.hex", 48, 64))
