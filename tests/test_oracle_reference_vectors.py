"""The oracle and the product's host code against vectors written from the reference itself.

tests/golden/make_reference_vectors.py imported the reference's numpy model once, in the
build container, and recorded what its own tb/vectors fixtures leave open: the
Codebook.gaussian integers at every width (config 4 uses 3-bit keys and values), one
collect() step at Llama-3-8B's attention shape with 3b/3b codes (d = 128, a 128-point
FWHT), one at config 0's context (512 + 1), and 40 decode steps from an empty cache.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

from oracle import native
from oracle.attention import attend_online, attend_two_pass, scores
from oracle.codebook import gaussian
from oracle.quantize import Cache, Format, encode, pack, unpack
from oracle.rotate import rotate, signs_from_seed

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def test_codebook_integers_at_every_width_equal_the_reference():
    """Codebook.gaussian(b), b = 1 .. 8 (ops/codebook.py:67-120), integer for integer:
    the oracle's restated Lloyd solve and the product's."""
    from insitu_amd.codebook import Codebook
    books = json.load(open(os.path.join(GOLD, "codebooks_gaussian.json")))["codebooks"]
    assert sorted(int(b) for b in books) == list(range(1, 9))
    for b, cb in books.items():
        c, bd = gaussian(int(b))
        np.testing.assert_array_equal(c, cb["centroids"], err_msg=f"oracle centroids, {b} bits")
        np.testing.assert_array_equal(bd, cb["boundaries"], err_msg=f"oracle boundaries, {b} bits")
        p = Codebook.gaussian(int(b))
        np.testing.assert_array_equal(p.centroids, cb["centroids"], err_msg=f"product, {b} bits")
        np.testing.assert_array_equal(p.boundaries, cb["boundaries"], err_msg=f"product, {b} bits")


STEPS = [("d128_3b3b_ctx64.npz", 128, 3, 3), ("d64_4b2b_ctx512.npz", 64, 4, 2)]


@pytest.mark.parametrize("name,d,kb,vb", STEPS, ids=["d128_3b3b", "d64_4b2b_ctx512"])
def test_one_step_every_stage(name, d, kb, vb):
    """Rotation, norms, codes and the packed row of the step's token, every cached row's
    scores, and attend_online / attend_two_pass over the whole cache, in numpy and in C."""
    z = _load(name)
    fmt = Format(d=d, key_bits=kb, value_bits=vb)
    kc, kbnd, vc, vbnd = fmt.codebooks()
    for got, key in ((kc, "key_centroids"), (kbnd, "key_bounds"), (vc, "value_centroids"),
                     (vbnd, "value_bounds")):
        np.testing.assert_array_equal(got, z[key])
    sg = signs_from_seed(d, 0, 1)
    for s in "qkv":
        np.testing.assert_array_equal(rotate(z[f"wire_{s}"][0], sg), z[f"rot_{s}"][0])
    row = pack(encode(z["rot_k"][0], z["rot_v"][0], fmt), fmt)
    np.testing.assert_array_equal(row, z["row"])
    cache = z["cache"]
    np.testing.assert_array_equal(cache[-1], z["row"])
    qr = z["rot_q"][0]
    on = np.zeros((32, d), dtype=np.int64)
    tp = np.zeros((32, d), dtype=np.int64)
    for h in range(8):
        kv = unpack(cache[:, h], fmt)
        q = qr[4 * h:4 * h + 4]
        s, _ = scores(q, kv, fmt)
        np.testing.assert_array_equal(s, z["scores"][4 * h:4 * h + 4])
        on[4 * h:4 * h + 4] = attend_online(q, kv, fmt)[0]
        tp[4 * h:4 * h + 4] = attend_two_pass(q, kv, fmt)[0]
        np.testing.assert_array_equal(native.attend_online(q, kv, fmt)[0], on[4 * h:4 * h + 4])
        np.testing.assert_array_equal(native.attend_two_pass(q, kv, fmt)[0], tp[4 * h:4 * h + 4])
    np.testing.assert_array_equal(on.reshape(-1), z["out_online"][0])
    np.testing.assert_array_equal(tp.reshape(-1), z["out_two_pass"][0])


def test_decode_steps_from_an_empty_cache():
    """40 steps from empty (kernel.py:256-353 per token): each appended row and each
    step's online output, the current token attending to itself."""
    z = _load("d64_4b2b_steps_from_empty.npz")
    fmt = Format()
    sg = signs_from_seed(64, 0, 1)
    n = z["wire_q"].shape[0]
    cache = Cache(8, n, fmt)
    for t in range(n):
        kr, vr = rotate(z["wire_k"][t], sg), rotate(z["wire_v"][t], sg)
        cache.append_rotated(kr[None], vr[None])
        np.testing.assert_array_equal(cache.buf[t], z["rows"][t], err_msg=f"row of step {t}")
        qr = rotate(z["wire_q"][t], sg)
        out = np.concatenate([attend_online(qr[4 * h:4 * h + 4], cache.view(h), fmt)[0]
                              for h in range(8)])
        np.testing.assert_array_equal(out.reshape(-1), z["out_online"][t], err_msg=f"step {t}")
    # and the C restatement of the same steps in one call
    heads = [unpack(cache.buf[:n, h], fmt) for h in range(8)]
    qrs = rotate(z["wire_q"].reshape(-1, 64), sg).reshape(n, 32, 64)
    got = native.decode_steps(qrs, heads, fmt)
    np.testing.assert_array_equal(got.reshape(n, -1), z["out_online"])
