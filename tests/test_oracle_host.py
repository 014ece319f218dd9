"""The host-half oracle (oracle/host.py) against the reference's goldens and closed forms."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import hexio as hx
from oracle import host
from oracle.quantize import Cache, Format
from oracle.rotate import matrix, rotate, signs_from_seed

HIDDEN, NQ, NKV, D = 2048, 32, 8, 64


def _golden_inputs():
    """hw/vectors.py:821-841 at ctx 64, seed 0: the seeded weights (weights.py:112-133,
    the kernel's default Weights.random(seed=0)), 64 context rows and the step row."""
    wq, wk, wv, _ = host.random_weights(HIDDEN, NQ, NKV, D, seed=0)
    w = np.concatenate([host.to_fp16(wq), host.to_fp16(wk), host.to_fp16(wv)])
    rng = np.random.default_rng(0)
    ctx_rows = rng.standard_normal((64, HIDDEN)).astype(np.float32) * 0.02
    step = rng.standard_normal((1, HIDDEN)).astype(np.float32) * 0.02
    return w, np.concatenate([ctx_rows, step])


@pytest.fixture(scope="module")
def golden_wire():
    w, x = _golden_inputs()
    cos, sin = host.rope_tables(D, 4096)              # build(): max_position 4096, theta 1e4
    p = host.project(w, x)
    # the board's order (cast_after_rope = False), which the golden vectors were taken in
    (q, k, v), sat = host.seam(p, NQ, NKV, D, np.arange(65), cos, sin, cast_after_rope=False)
    return q, k, v, sat


def test_step_wire_rows_are_the_golden_vectors(golden_wire):
    q, k, v, sat = golden_wire
    np.testing.assert_array_equal(q[64], hx.lanes("wire_q.hex", 24).reshape(NQ, D))
    np.testing.assert_array_equal(k[64], hx.lanes("wire_k.hex", 24).reshape(NKV, D))
    np.testing.assert_array_equal(v[64], hx.lanes("wire_v.hex", 24).reshape(NKV, D))
    assert sat == 0


def test_all_65_cached_rows_follow_from_the_host_half(golden_wire):
    """Positions 0 .. 64 through rotate, encode and pack give the cache_rows fixtures."""
    _, k, v, _ = golden_wire
    sg = signs_from_seed(D, 0, 1)
    c = Cache(NKV, 65, Format())
    c.append_rotated(rotate(k, sg), rotate(v, sg))
    rows = np.stack([hx.bytes_rows(f"cache_rows_h{h}.hex") for h in range(NKV)], axis=1)
    np.testing.assert_array_equal(c.buf, rows)


def test_cast_orders_differ_by_the_casts_rounding():
    """RoPE in float before the cast or in fixed point after it: the cast's half-LSB
    goes through the rotation (|c| + |s| <= sqrt 2) and the floor adds one: <= 2 LSB."""
    w, x = _golden_inputs()
    cos, sin = host.rope_tables(D, 4096)
    p = host.project(w, x)
    a, _ = host.seam(p, NQ, NKV, D, np.arange(65), cos, sin, cast_after_rope=True)
    b, _ = host.seam(p, NQ, NKV, D, np.arange(65), cos, sin, cast_after_rope=False)
    for ta, tb in zip(a, b):
        assert np.abs(ta - tb).max() <= 2
    np.testing.assert_array_equal(a[2], b[2])            # V carries no position


def test_to_fixed_rounds_half_to_even_and_saturates():
    lsb = 1.0 / 65536
    codes, sat = host.to_fixed(np.array([0.5, 1.5, 2.5, -0.5, -1.5]) * lsb)
    np.testing.assert_array_equal(codes, [0, 2, 2, 0, -2])
    assert sat == 0
    codes, sat = host.to_fixed(np.array([200.0, -200.0, 127.99998]))
    np.testing.assert_array_equal(codes, [(1 << 23) - 1, -(1 << 23), 8388607])
    assert sat == 2


def test_rope_table_and_position_zero():
    cos, sin = host.rope_tables(D, 8)
    assert np.all(cos[0] == 1 << 15) and np.all(sin[0] == 0)
    x = np.random.default_rng(1).integers(-(1 << 20), 1 << 20, size=(3, D))
    np.testing.assert_array_equal(host.rope_fixed(x, np.zeros(3, dtype=np.int64), cos, sin), x)
    # one channel pair at position 1: the textbook 2-D rotation by inv_freq[0] = 1 rad,
    # to the Q15 table's half-LSB (2^-16, 16 units at 2^20) and the floor
    e = np.zeros(D, dtype=np.int64)
    e[0] = 1 << 20
    y = host.rope_fixed(e, 1, cos, sin)
    assert abs(y[0] - (1 << 20) * np.cos(1.0)) <= 17
    assert abs(y[D // 2] - (1 << 20) * np.sin(1.0)) <= 17


# Llama-3.2-1B's rope_scaling (the reference's test_rope_scaling.py properties)
S = host.RopeScaling(factor=32.0, low_freq_factor=1.0, high_freq_factor=4.0, original_max_position=8192)


def _inv_freq(theta=500000.0):
    return 1.0 / (theta ** (np.arange(0, D // 2, dtype=np.float64) * 2.0 / D))


def test_rope_scaling_regimes():
    f = _inv_freq()
    out = S.apply(f)
    wavelen = 2.0 * np.pi / f
    short = wavelen < S.original_max_position / S.high_freq_factor
    long = wavelen > S.original_max_position / S.low_freq_factor
    assert short.any() and long.any()
    np.testing.assert_array_equal(out[short], f[short])
    np.testing.assert_allclose(out[long], f[long] / S.factor)
    assert np.all(out <= f * (1 + 1e-12)) and np.all(out >= f / S.factor * (1 - 1e-12))
    assert np.all(np.diff(out / f) <= 1e-12)
    plain = host.rope_tables(D, 64, 500000.0)
    scaled = host.rope_tables(D, 64, 500000.0, scaling=S)
    assert not np.array_equal(plain[0], scaled[0])
    np.testing.assert_array_equal(plain[0][0], scaled[0][0])
    with pytest.raises(ValueError):
        host.RopeScaling(factor=8.0, low_freq_factor=4.0, high_freq_factor=1.0, original_max_position=8192)


def test_fold_undoes_the_rotation():
    """W_o' = W_o blockdiag(R^-1): applying W_o' to rotated heads is W_o on the originals."""
    sg = signs_from_seed(D, 0, 1)
    rng = np.random.default_rng(4)
    wo = rng.standard_normal((16, 2 * D))
    folded = host.fold_o_proj(wo, sg, 2)
    r = matrix(sg)
    x = rng.standard_normal((3, 2 * D))
    xr = np.concatenate([x[:, :D] @ r.T, x[:, D:] @ r.T], axis=1)     # each head rotated
    np.testing.assert_allclose(xr @ folded.T, x @ wo.T, rtol=1e-12, atol=1e-12)
