"""GPU parity of the host half (kernel.py:198-249) and the output side (:348-356).

The casts and the seam epilogue are exact against the oracle: for the GPU's own
fp32 projections, the wire rows are oracle/host.py's integers bit for bit, in
both cast orders. The projections themselves are fp16 GEMMs whose fp32 sums run
in rocBLAS's order, not numpy's; the reference states that its own functional
and hardware modes differ the same way (ops/project.py:6-11). They are held to
the worst-case bound of an fp32 sum of K exact fp16 products, checked per
element against the float64 sum: |y - exact| <= 2 K 2^-24 sum |w x|.
"""

import numpy as np
import pytest

from oracle import hexio as hx
from oracle import host as oh
from oracle import native
from oracle.quantize import Cache, Format
from oracle.rotate import matrix, rotate, signs_from_seed

pytestmark = pytest.mark.gpu

HIDDEN, NQ, NKV, D = 2048, 32, 8, 64
FMT = Format()


def _golden_inputs():
    """hw/vectors.py:821-841 at ctx 64, seed 0: 64 context rows and the step row."""
    rng = np.random.default_rng(0)
    ctx_rows = rng.standard_normal((64, HIDDEN)).astype(np.float32) * 0.02
    step = rng.standard_normal((1, HIDDEN)).astype(np.float32) * 0.02
    return np.concatenate([ctx_rows, step])


def _check_gemm(y, w, x, bias=None):
    """y (n, out) against the float64 sum of the fp16 products, to the fp32 bound."""
    w16 = oh.to_fp16(w).astype(np.float64)
    x16 = oh.to_fp16(x).astype(np.float64)
    exact = x16 @ w16.T
    mag = np.abs(x16) @ np.abs(w16).T
    tol = 2.0 * w16.shape[1] * 2.0 ** -24 * mag
    if bias is not None:
        exact = exact + np.asarray(bias, np.float32).astype(np.float64)
        tol = tol + np.abs(exact) * 2.0 ** -23
    err = np.abs(np.asarray(y, np.float64) - exact)
    assert np.all(err <= tol + 1e-30), f"max excess {np.max(err - tol)}"
    return err


def _model(**kw):
    from insitu_amd import ModelConfig
    return ModelConfig(hidden_size=HIDDEN, num_heads=NQ, num_kv_heads=NKV, head_dim=D, **kw)


@pytest.fixture(scope="module")
def golden_half(ctx):
    from insitu_amd.host import HostHalf, Weights
    model = _model()
    w = Weights.random(model, matrix(signs_from_seed(D, 0, 1)), seed=0, ctx=ctx)
    return model, w, HostHalf(model, w, cast_after_rope=False, ctx=ctx)


def test_seeded_weights_are_the_oracles(golden_half):
    """weights.py:112-133 through Weights.random: the oracle's arrays, cast to fp16."""
    _, w, _ = golden_half
    wq, wk, wv, wo = oh.random_weights(HIDDEN, NQ, NKV, D, seed=0)
    got = w.qkv.cpu().numpy().view(np.float16)
    np.testing.assert_array_equal(got, oh.to_fp16(np.concatenate([wq, wk, wv])))
    folded = oh.fold_o_proj(wo, signs_from_seed(D, 0, 1), NQ)
    got_o = w.o.cpu().numpy().view(np.float16).astype(np.float64)
    # the fold in float64, then one cast to fp16: a half-ulp apart at most
    np.testing.assert_allclose(got_o, oh.to_fp16(folded).astype(np.float64), rtol=2.0 ** -10, atol=2.0 ** -24)


@pytest.mark.parametrize("n", [5, 3, 1])
def test_fp16_casts_are_exact_through_an_identity_gemm(ctx, n):
    """W = I makes the GEMM exact, so y is the staging cast itself: fp32 -> fp16
    half to even (numerics/fp.py:20-22) and Q16 -> float64 -> fp16 in one rounding.
    n = 5 tokens run the cast kernel and rocBLAS, n <= 4 the decode GEMV."""
    import torch
    from insitu_amd import _lib
    from insitu_amd.runtime import ptr
    n_in = 256
    eye = torch.from_numpy(np.eye(n_in, dtype=np.float16).view(np.int16)).to(ctx.torch_device)
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((5, n_in)) * np.exp2(rng.integers(-20, 13, (5, n_in)))).astype(np.float32)
    x[0, :8] = [1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, -(1.0 + 2.0 ** -11), 65504.0, 2.0 ** -24,
                2.0 ** -25, 3 * 2.0 ** -25, 0.0]                  # ties, the top, subnormals
    x = np.ascontiguousarray(x[:n])
    bias = rng.standard_normal(n_in).astype(np.float32)
    xd = torch.from_numpy(x).to(ctx.torch_device)
    bd = torch.from_numpy(bias).to(ctx.torch_device)
    y = torch.empty((n, n_in), dtype=torch.float32, device=ctx.torch_device)
    _lib.check(ctx.lib.insitu_project(ctx.handle, ptr(eye), n_in, n_in, ptr(xd), n, None, ptr(y)))
    np.testing.assert_array_equal(y.cpu().numpy(), oh.to_fp16(x).astype(np.float32))
    _lib.check(ctx.lib.insitu_project(ctx.handle, ptr(eye), n_in, n_in, ptr(xd), n, ptr(bd), ptr(y)))
    np.testing.assert_array_equal(y.cpu().numpy(), oh.to_fp16(x).astype(np.float32) + bias)

    q16 = rng.integers(-(1 << 31), (1 << 31) - 1, size=(5, n_in), dtype=np.int64)
    q16[0, :6] = [1, -1, 0, (1 << 31) - 1, -(1 << 31), 65536 + 32]   # 1 + 2^-11: a tie to even
    q16[1] = rng.integers(-(1 << 18), 1 << 18, n_in)
    q16 = np.ascontiguousarray(q16[:n])
    qd = torch.from_numpy(q16.astype(np.int32)).to(ctx.torch_device)
    _lib.check(ctx.lib.insitu_output_projection(ctx.handle, ptr(qd), n, n_in, 16, ptr(eye), n_in, None, ptr(y)))
    want = oh.to_fp16(q16.astype(np.float64) / 65536.0).astype(np.float32)
    np.testing.assert_array_equal(y.cpu().numpy(), want)


def test_projections_within_the_fp32_bound(golden_half):
    _, w, half = golden_half
    wq, wk, wv, _ = oh.random_weights(HIDDEN, NQ, NKV, D, seed=0)
    x = _golden_inputs()
    p = half.project_qkv(x).cpu().numpy()
    _check_gemm(p, np.concatenate([wq, wk, wv]), x)
    for n in (1, 2, 4):                                   # the decode GEMV
        _check_gemm(half.project_qkv(x[:n]).cpu().numpy(), np.concatenate([wq, wk, wv]), x[:n])
    # and against the oracle's float32 numpy product, to a few ulp
    ref = oh.project(np.concatenate([wq, wk, wv]), x)
    np.testing.assert_allclose(p, ref, rtol=0, atol=1e-6)


@pytest.mark.parametrize("cast_after_rope", [True, False])
@pytest.mark.parametrize("scaled", [False, True])
def test_seam_epilogue_is_exact_on_the_gpus_projections(ctx, cast_after_rope, scaled):
    """split heads, q * 1/sqrt(d), RoPE and the cast (kernel.py:209-249) on the
    GPU's own fp32 projections: the oracle's wire integers and saturation count
    exactly, with biases, Llama 3 RoPE scaling, positions across the table and
    rows large enough to saturate."""
    from insitu_amd.host import HostHalf, RopeScaling, Weights
    kw = {}
    if scaled:
        kw = dict(rope_theta=500000.0, max_position=8192,
                  rope_scaling=RopeScaling(32.0, 1.0, 4.0, 8192))
    model = _model(**kw)
    rng = np.random.default_rng(11)
    n = 40
    biases = [rng.standard_normal(m).astype(np.float32) * 0.05 for m in (NQ * D, NKV * D, NKV * D)]
    wq, wk, wv, wo = oh.random_weights(HIDDEN, NQ, NKV, D, seed=3)
    w = Weights(wq, wk, wv, wo, model, matrix(signs_from_seed(D, 0, 1)), q_bias=biases[0],
                k_bias=biases[1], v_bias=biases[2], ctx=ctx)
    half = HostHalf(model, w, cast_after_rope=cast_after_rope, ctx=ctx)
    x = (rng.standard_normal((n, HIDDEN)) * np.logspace(-2, 3.5, n)[:, None]).astype(np.float32)
    pos = rng.integers(0, model.max_position, n)
    pos[:3] = [0, model.max_position - 1, 1]
    q, k, v = half.wire(x, pos)
    p = half.project_qkv(x).cpu().numpy()                  # the same fp32 projections, again
    cos, sin = oh.rope_tables(D, model.max_position, model.rope_theta,
                              scaling=oh.RopeScaling(32.0, 1.0, 4.0, 8192) if scaled else None)
    np.testing.assert_array_equal(half.rope.cos, cos)
    np.testing.assert_array_equal(half.rope.sin, sin)
    (wq_, wk_, wv_), sat = oh.seam(p, NQ, NKV, D, pos, cos, sin, bias=np.concatenate(biases),
                                   cast_after_rope=cast_after_rope)
    np.testing.assert_array_equal(q.cpu().numpy(), wq_)
    np.testing.assert_array_equal(k.cpu().numpy(), wk_)
    np.testing.assert_array_equal(v.cpu().numpy(), wv_)
    assert sat > 0 and half.last_saturated == sat


def test_golden_wire_rows_from_the_hidden_states(golden_half):
    """hw/vectors.py:821-841: the step row's wire q/k/v from seeded weights and
    hidden states, the board's cast order. rocBLAS's fp32 sums may round a lane
    the other way: at most 2 LSB (one for the cast, one through RoPE), rarely."""
    _, _, half = golden_half
    x = _golden_inputs()
    q, k, v = (t.cpu().numpy() for t in half.wire(x, np.arange(65)))
    for got, name, heads in ((q, "q", NQ), (k, "k", NKV), (v, "v", NKV)):
        want = hx.lanes(f"wire_{name}.hex", 24).reshape(heads, D)
        diff = np.abs(got[64].astype(np.int64) - want)
        assert diff.max() <= 2, name
        assert np.count_nonzero(diff) <= max(2, want.size // 200), name
    assert half.last_saturated == 0


def test_position_beyond_the_table_raises(golden_half):
    from insitu_amd._lib import FormatError
    _, _, half = golden_half
    with pytest.raises(FormatError):
        half.wire(_golden_inputs()[:2], [3, 4096])


def test_output_side_within_the_fp32_bound(golden_half):
    _, w, half = golden_half
    rng = np.random.default_rng(5)
    out = rng.integers(-(1 << 19), 1 << 19, size=(9, NQ * D))
    y = half.output(out).cpu().numpy()
    wo = w.o.cpu().numpy().view(np.float16)
    _check_gemm(y, wo, out / 65536.0)
    for n in (1, 3):                                      # the decode GEMV
        _check_gemm(half.output(out[:n]).cpu().numpy(), wo, out[:n] / 65536.0)
    # the oracle's output side (float32 numpy sums) agrees to a few ulp
    np.testing.assert_allclose(y, oh.output_side(out, wo), rtol=0, atol=2e-5 * np.abs(y).max())


@pytest.mark.parametrize("cast_after_rope", [False, True])
def test_forward_hidden_states_end_to_end(ctx, golden_half, cast_after_rope):
    """kernel.py:177-357 through AttentionBlock.forward: a 64-token prompt, then a
    decode step. The wire taps equal the oracle's seam on the GPU's projections;
    the Q16 out tap equals the oracle's seam half (rotate, encode, attend) run on
    those wire rows; y is the output side of that tap, to the fp32 bound."""
    from insitu_amd import AttentionBlock, QuantConfig
    model, w, _ = golden_half
    blk = AttentionBlock(model, QuantConfig(key_bits=4, value_bits=2), capacity=80, weights=w,
                         cast_after_rope=cast_after_rope, ctx=ctx)
    x = _golden_inputs()
    y0, r0 = blk.forward(x[:64])
    taps0 = {k: t.cpu().numpy() for k, t in blk.taps.items()}
    y1, r1 = blk.forward(x[64])
    taps1 = {k: t.cpu().numpy() for k, t in blk.taps.items()}
    assert (r0.n_tokens, r0.context, r1.n_tokens, r1.context) == (64, 64, 1, 65)
    wire = {k: np.concatenate([taps0[k], taps1[k]]) for k in ("wire.q", "wire.k", "wire.v")}

    # the prompt's projections ran as one GEMM, the decode step's as the GEMV
    p = np.concatenate([blk.host.project_qkv(x[:64]).cpu().numpy(), blk.host.project_qkv(x[64:]).cpu().numpy()])
    cos, sin = oh.rope_tables(D, model.max_position)
    (wq_, wk_, wv_), _ = oh.seam(p, NQ, NKV, D, np.arange(65), cos, sin, cast_after_rope=cast_after_rope)
    np.testing.assert_array_equal(wire["wire.q"], wq_)
    np.testing.assert_array_equal(wire["wire.k"], wk_)
    np.testing.assert_array_equal(wire["wire.v"], wv_)

    sg = signs_from_seed(D, 0, 1)
    cache = Cache(NKV, 65, FMT)
    cache.append_rotated(rotate(wk_, sg), rotate(wv_, sg))
    np.testing.assert_array_equal(blk.cache.buf[:65], cache.buf)
    want = native.decode_steps(rotate(wq_, sg), [cache.view(h) for h in range(NKV)], FMT)
    out = np.concatenate([taps0["out"], taps1["out"]])
    np.testing.assert_array_equal(out, want.reshape(65, NQ * D))

    y = np.concatenate([y0.cpu().numpy(), y1.cpu().numpy()])
    _check_gemm(y, w.o.cpu().numpy().view(np.float16), out / 65536.0)


def test_two_contexts_on_one_device_keep_their_own_blas_state(ctx, golden_half):
    """Each context has its own rocBLAS handle, fp16 staging and counters: two contexts
    on two streams of one device, used in turn with prompts of different lengths (the
    staging grows), give the single-context results and their own saturation counts,
    and destroying one leaves the other working."""
    import torch
    from insitu_amd.host import HostHalf, Weights
    from insitu_amd.runtime import Context
    model, _, _ = golden_half
    rng = np.random.default_rng(5)
    xs = [(rng.standard_normal((n, HIDDEN)) * s).astype(np.float32)
          for n, s in ((3, 0.02), (40, 50.0), (7, 0.02), (65, 50.0))]
    pos = [np.arange(x.shape[0]) for x in xs]
    ref = []
    w0 = Weights.random(model, matrix(signs_from_seed(D, 0, 1)), seed=0, ctx=ctx)
    h0 = HostHalf(model, w0, cast_after_rope=False, ctx=ctx)
    for x, p in zip(xs, pos):
        q, k, v = (t.cpu().numpy() for t in h0.wire(x, p))
        ref.append((q, k, v, h0.last_saturated))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    ctxs = [Context(0, s) for s in streams]
    halves = []
    for c, s in zip(ctxs, streams):
        with torch.cuda.stream(s):
            w = Weights.random(model, matrix(signs_from_seed(D, 0, 1)), seed=0, ctx=c)
            halves.append(HostHalf(model, w, cast_after_rope=False, ctx=c))
    for i, (x, p) in enumerate(zip(xs, pos)):
        for j in (i % 2, 1 - i % 2):
            with torch.cuda.stream(streams[j]):
                q, k, v = halves[j].wire(x, p)
                got = (q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(), halves[j].last_saturated)
            for a, b in zip(got[:3], ref[i][:3]):
                np.testing.assert_array_equal(a, b, err_msg=f"prompt {i}, context {j}")
            assert got[3] == ref[i][3] and (ref[i][3] > 0) == (i % 2 == 1), (i, j)
    torch.cuda.synchronize()
    ctxs[0].close()
    with torch.cuda.stream(streams[1]):
        q, _, _ = halves[1].wire(xs[3], pos[3])
        np.testing.assert_array_equal(q.cpu().numpy(), ref[3][0])


@pytest.mark.parametrize("cast_after_rope", [True, False])
@pytest.mark.parametrize("n", [1, 2, 4])
def test_fused_decode_seam_is_exact_on_its_projections(ctx, cast_after_rope, n):
    """insitu_project_seam for a decode step (n <= 4 tokens: gemv_seam_kernel, the last
    workgroup of each head running its seam): the wire rows are the oracle's seam of the
    projections the same call wrote, bit for bit, with biases, positions across the table
    (given, and consecutive from pos0) and saturating rows; the projections within the
    fp32 bound."""
    import ctypes
    import torch
    from insitu_amd import _lib
    from insitu_amd.host import ROPE_FRAC, HostHalf, Weights
    from insitu_amd.runtime import ptr
    model = _model()
    rng = np.random.default_rng(50 + n)
    biases = [rng.standard_normal(m).astype(np.float32) * 0.05 for m in (NQ * D, NKV * D, NKV * D)]
    wq, wk, wv, wo = oh.random_weights(HIDDEN, NQ, NKV, D, seed=5)
    w = Weights(wq, wk, wv, wo, model, matrix(signs_from_seed(D, 0, 1)), q_bias=biases[0],
                k_bias=biases[1], v_bias=biases[2], ctx=ctx)
    half = HostHalf(model, w, cast_after_rope=cast_after_rope, ctx=ctx)
    cos, sin = oh.rope_tables(D, model.max_position, model.rope_theta)
    for trial, scale in enumerate((0.02, 300.0, 3000.0)):      # the last ones saturate
        x = (rng.standard_normal((n, HIDDEN)) * scale).astype(np.float32)
        for consecutive in (False, True):
            pos = (np.arange(n) + [7, model.max_position - n][trial % 2]) if consecutive else \
                rng.integers(0, model.max_position, n)
            q, k, v = half.wire(x, pos)
            p = half._keep[1].cpu().numpy()
            _check_gemm(p, np.concatenate([wq, wk, wv]), x)
            (wq_, wk_, wv_), sat = oh.seam(p, NQ, NKV, D, pos, cos, sin, bias=np.concatenate(biases),
                                           cast_after_rope=cast_after_rope)
            np.testing.assert_array_equal(q.cpu().numpy(), wq_)
            np.testing.assert_array_equal(k.cpu().numpy(), wk_)
            np.testing.assert_array_equal(v.cpu().numpy(), wv_)
            assert half.last_saturated == sat
            if trial:
                assert sat > 0
    np.testing.assert_array_equal(half.rope.cos, cos)
    # a position beyond the table, found on the device: ERANGE, and the per-head tickets
    # are left ready for the next call
    from insitu_amd._lib import FormatError
    dev = ctx.torch_device
    xd = torch.from_numpy(x).to(dev)
    bad = torch.from_numpy(np.full(n, model.max_position, np.int64)).to(dev)
    pd = torch.empty((n, (NQ + 2 * NKV) * D), dtype=torch.float32, device=dev)
    qd = torch.empty((n, NQ, D), dtype=torch.int32, device=dev)
    kd = torch.empty((n, NKV, D), dtype=torch.int32, device=dev)
    vd = torch.empty((n, NKV, D), dtype=torch.int32, device=dev)
    cnt = (ctypes.c_uint64 * 2)()
    bias = w.qkv_bias
    with pytest.raises(FormatError):
        _lib.check(ctx.lib.insitu_project_seam(
            ctx.handle, ptr(w.qkv), HIDDEN, ptr(xd), n, ptr(bias), NQ, NKV, D, ptr(bad), 0,
            ptr(half._cos), ptr(half._sin), model.max_position, ROPE_FRAC, half.attn_scale,
            1 if cast_after_rope else 0, ptr(pd), ptr(qd), ptr(kd), ptr(vd), cnt))
    assert cnt[1] == n * (NQ + NKV)                 # every q and k row of every token
    q2, _, _ = half.wire(x, np.arange(n))
    p = half._keep[1].cpu().numpy()
    (wq_, _, _), _ = oh.seam(p, NQ, NKV, D, np.arange(n), cos, sin, bias=np.concatenate(biases),
                             cast_after_rope=cast_after_rope)
    np.testing.assert_array_equal(q2.cpu().numpy(), wq_)
