"""GPU: the boundary the reference's callers use.

1. The torch adapter (insitu_amd.adapters.torch_llama), against a stub attention
   module shaped like tests/test_adapter.py:23-97 of the reference (shapes, dtypes,
   2-D input, the batch guard, nn.Module, the report and reset), and against a
   small random transformers LlamaForCausalLM (no download): the decoder layer's
   real call (position_ids, past_key_values advanced), graft / ungraft, greedy
   generation with every layer grafted, and the grafted layer's Q16 output equal
   to the oracle's attend on its own wire rows.
2. The seam as kernel.py:280-345 drives it: cache.append_rotated(kr, vr, trace),
   cache.view(h, trace, n_reads=n) into attend_online_batch / attend_causal_batch,
   cache.view(h, trace).select(slice(0, ctx)) into attend_online / attend_two_pass,
   each against the oracle on the same rows.
"""

import numpy as np
import pytest

from oracle import native
from oracle.quantize import Cache, Format
from oracle.rotate import rotate, signs_from_seed

pytestmark = pytest.mark.gpu


class _StubConfig:
    # the reference stub's shape with head_dim 64 (the kernels take 64 and 128)
    hidden_size = 256
    num_attention_heads = 4
    num_key_value_heads = 2
    head_dim = 64
    rope_theta = 10000.0
    max_position_embeddings = 256


class _StubAttention:
    """Just enough of a Llama attention module to be read for its weights."""

    def __init__(self):
        import torch
        import torch.nn as nn
        torch.manual_seed(0)
        c = _StubConfig
        self.q_proj = nn.Linear(c.hidden_size, c.num_attention_heads * c.head_dim, bias=False)
        self.k_proj = nn.Linear(c.hidden_size, c.num_key_value_heads * c.head_dim, bias=False)
        self.v_proj = nn.Linear(c.hidden_size, c.num_key_value_heads * c.head_dim, bias=False)
        self.o_proj = nn.Linear(c.num_attention_heads * c.head_dim, c.hidden_size, bias=False)


def _stub_adapter(ctx):
    from insitu_amd.adapters.torch_llama import build_from_layer
    return build_from_layer(_StubAttention(), _StubConfig, capacity=64, ctx=ctx)


def test_adapter_shapes_and_dtype(ctx):
    import torch
    a = _stub_adapter(ctx)
    x = torch.randn(1, 5, 256)
    y, weights = a(x)
    assert y.shape == x.shape and y.dtype == x.dtype and weights is None
    assert y.device == x.device
    y16, _ = a(torch.randn(1, 2, 256, dtype=torch.float16))
    assert y16.dtype == torch.float16


def test_adapter_accepts_two_dim_input(ctx):
    import torch
    a = _stub_adapter(ctx)
    y, _ = a(torch.randn(3, 256))
    assert y.shape == (3, 256)


def test_adapter_refuses_a_padded_batch(ctx):
    import torch
    a = _stub_adapter(ctx)
    with pytest.raises(NotImplementedError, match="batch of 2"):
        a(torch.randn(2, 5, 256))


def test_adapter_is_an_nn_module(ctx):
    import torch.nn as nn
    assert isinstance(_stub_adapter(ctx), nn.Module)


def test_adapter_carries_a_report(ctx):
    import torch
    a = _stub_adapter(ctx)
    a(torch.randn(1, 4, 256))
    assert a.last_report is not None and a.last_report.context == 4
    a.reset()
    a(torch.randn(1, 2, 256))
    assert a.last_report.context == 2


def test_adapter_refuses_what_it_does_not_model(ctx):
    import torch.nn as nn
    from insitu_amd.adapters.torch_llama import build_from_layer
    with pytest.raises(NotImplementedError):
        build_from_layer(_StubAttention(), _StubConfig, compressed=False, ctx=ctx)
    m = _StubAttention()
    m.q_norm = nn.LayerNorm(64)
    m.k_norm = nn.LayerNorm(64)
    with pytest.raises(NotImplementedError, match="QK-norm"):
        build_from_layer(m, _StubConfig, ctx=ctx)


# -- a transformers Llama, random weights --------------------------------------------

def _llama(layers=2):
    import torch
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(1)
    cfg = LlamaConfig(hidden_size=512, intermediate_size=768, num_attention_heads=8,
                      num_key_value_heads=2, head_dim=64, num_hidden_layers=layers, vocab_size=256,
                      max_position_embeddings=512, rope_theta=10000.0)
    model = LlamaForCausalLM(cfg).eval()
    return model


def test_grafted_layer_output_is_the_oracles_on_its_wire_rows(ctx):
    """Layer 1 grafted (8 query heads over 2 KV heads, d = 64): after a prompt and
    two decode steps through the whole model, the block's last Q16 output equals the
    oracle's attend_online over the rows the block appended, for the query the block
    put on the wire (the GPU's own projections: below the seam, bit for bit)."""
    import torch
    from insitu_amd import QuantConfig
    from insitu_amd.adapters.torch_llama import graft, ungraft
    from transformers import DynamicCache
    model = _llama()
    orig = graft(model, [1], quant=QuantConfig(key_bits=4, value_bits=2), softmax="online", ctx=ctx)
    adapter = model.model.layers[1].self_attn
    ids = torch.tensor([[3, 17, 250, 8, 99, 41, 7]])
    cache = DynamicCache()
    with torch.no_grad():
        out = model(input_ids=ids, past_key_values=cache, use_cache=True)
        for t in range(2):
            nxt = out.logits[:, -1:].argmax(-1)
            out = model(input_ids=nxt, past_key_values=cache, use_cache=True)
            assert cache.get_seq_length() == ids.shape[1] + t + 1
    blk = adapter.kernel
    assert blk.cache.length == ids.shape[1] + 2 == adapter.last_report.context
    f = Format(d=64, key_bits=4, value_bits=2)
    sg = signs_from_seed(64, 0, 1)
    qr = rotate(blk.taps["wire.q"].cpu().numpy().reshape(8, 64).astype(np.int64), sg)
    want = np.concatenate([native.attend_online(qr[4 * h:4 * h + 4], blk.cache.view(h), f)[0]
                           for h in range(2)]).reshape(-1)
    np.testing.assert_array_equal(blk.taps["out"].cpu().numpy().reshape(-1), want)
    ungraft(model, orig)
    assert model.model.layers[1].self_attn is orig[1]


def test_graft_every_layer_and_generate(ctx):
    """Every layer grafted: the model's own length bookkeeping stays right (the
    adapter advances past_key_values), generation runs, and the logits stay close
    to the original model's at near-lossless codes (8-bit keys and values), where any
    large residual would be plumbing: a RoPE convention, a head layout, a fold."""
    import torch
    from insitu_amd import QuantConfig
    from insitu_amd.adapters.torch_llama import graft, ungraft
    model = _llama()
    ids = torch.tensor([[5, 9, 200, 31, 77, 2, 140, 18, 66, 4]])
    with torch.no_grad():
        ref = model(input_ids=ids).logits[0].float().numpy()
    orig = graft(model, [0, 1], quant=QuantConfig(key_bits=8, value_bits=8), capacity=64, ctx=ctx)
    with torch.no_grad():
        got = model(input_ids=ids).logits[0].float().numpy()
    for i in (0, 1):
        model.model.layers[i].self_attn.reset()
    with torch.no_grad():
        gen = model.generate(ids, max_new_tokens=6, do_sample=False)
    assert gen.shape == (1, ids.shape[1] + 6)
    assert model.model.layers[0].self_attn.kernel.cache.length == ids.shape[1] + 5
    ungraft(model, orig)
    cos = (ref * got).sum(-1) / (np.linalg.norm(ref, axis=-1) * np.linalg.norm(got, axis=-1))
    assert cos.min() > 0.99, cos
    with torch.no_grad():
        again = model(input_ids=ids).logits[0].float().numpy()
    np.testing.assert_array_equal(again, ref)


def test_compare_against_original_on_one_layer(ctx):
    """torch_llama.py:226-253 on captured hidden states with the layer's own
    position embeddings: near-lossless codes give a cosine near 1."""
    import torch
    from insitu_amd import QuantConfig
    from insitu_amd.adapters import torch_llama as tl
    model = _llama()
    torch.manual_seed(3)
    x = torch.randn(1, 12, 512) * 0.5
    pos = torch.arange(12)[None]
    with torch.no_grad():
        pe = model.model.rotary_emb(x, pos)
    layer = model.model.layers[0]
    with torch.no_grad():
        ref = layer.self_attn(x, position_embeddings=pe, attention_mask=None, position_ids=pos)[0]
    a = tl.build_from_layer(layer.self_attn, model.config, quant=QuantConfig(key_bits=8, value_bits=8),
                            ctx=ctx)
    with torch.no_grad():
        got = a(x, position_embeddings=pe, attention_mask=None, position_ids=pos)[0]
    r, g = ref.numpy().ravel(), got.numpy().ravel()
    cos = float(r @ g / (np.linalg.norm(r) * np.linalg.norm(g)))
    assert cos > 0.995, cos
    res = tl.compare_against_original(model, 0, x, position_embeddings=pe, attention_mask=None,
                                      position_ids=pos)
    assert res["cosine"] > 0.9 and res["report"].context == 12


# -- the seam, as kernel.py calls it -----------------------------------------------------

@pytest.mark.parametrize("softmax", ["online", "two_pass"])
def test_kernel_py_call_shapes_on_the_device_cache(ctx, softmax):
    """kernel.py:280-345 with this build's CompressedCache and CompressedAttention in
    place of the reference's: a prompt of 9 tokens (the batched path), then 3 decode
    tokens (the per-token path, view(h).select(slice(0, ctx))), each KV group's
    output equal to the oracle's on the same rows, and the statistics summed the
    reference's way (AttentionStats.merge)."""
    from insitu_amd import QuantConfig
    from insitu_amd.attention import AttentionStats, CompressedAttention
    from insitu_amd.cache import CompressedCache, DeviceKV
    rng = np.random.default_rng(8)
    n_kv, G, d, cap = 2, 4, 64, 40
    f = Format(d=d, key_bits=4, value_bits=2)
    cache = CompressedCache(n_kv, d, cap, QuantConfig(key_bits=4, value_bits=2), n_q_heads=n_kv * G, ctx=ctx)
    attn = CompressedAttention(cache)
    assert attn.score_mode == "fused"
    host = Cache(n_kv, cap, f)
    trace = object()                       # passed through, never touched

    def wire(n):
        return (rng.integers(-(1 << 22), 1 << 22, size=(n, n_kv * G, d)),
                rng.integers(-(1 << 22), 1 << 22, size=(n, n_kv, d)),
                rng.integers(-(1 << 22), 1 << 22, size=(n, n_kv, d)))

    fn = native.attend_online if softmax == "online" else native.attend_two_pass
    # prefill, kernel.py:316-331
    qr, kr, vr = wire(9)
    base = cache.length
    cache.append_rotated(kr, vr, trace)
    host.append_rotated(kr, vr)
    report = AttentionStats()
    for kvh in range(n_kv):
        heads = slice(kvh * G, (kvh + 1) * G)
        kv = cache.view(kvh, trace, n_reads=9)
        assert isinstance(kv, DeviceKV) and kv.n_tokens == 9
        if softmax == "online":
            y, st = attn.attend_online_batch(qr[:, heads], kv, base=base, trace=trace)
        else:
            y, st = attn.attend_causal_batch(qr[:, heads], kv, base=base, tile=256, trace=trace)
        report.merge(st)
        for i in range(9):
            want, _ = fn(qr[i, heads], host.view(kvh).select(slice(0, base + i + 1)), f)
            np.testing.assert_array_equal(y[i], want, err_msg=f"prompt token {i}, KV head {kvh}")
    assert report.n_tokens == 9
    # decode, kernel.py:333-341 and 383-392
    for t in range(3):
        qr, kr, vr = wire(1)
        base = cache.length
        cache.append_rotated(kr, vr, trace)
        host.append_rotated(kr, vr)
        ctx_len = base + 1
        for kvh in range(n_kv):
            heads = slice(kvh * G, (kvh + 1) * G)
            kv = cache.view(kvh, trace).select(slice(0, ctx_len))
            q = qr[0, heads]
            if softmax == "online":
                y, st = attn.attend_online(q, kv, trace)
                y = y.reshape(np.shape(q))
            else:
                y, st = attn.attend_two_pass(q, kv, trace)
            want, wst = fn(q, host.view(kvh).select(slice(0, ctx_len)), f)
            np.testing.assert_array_equal(y, want, err_msg=f"step {t}, KV head {kvh}")
            assert (st.rescale_events, st.max_abs_acc, st.n_tokens) == \
                (wst.rescale_events, wst.max_abs_acc, wst.n_tokens)
    # an earlier prefix of the same view: the context a token saw
    kv = cache.view(1).select(slice(0, 5))
    y, _ = attn.attend_online(qr[0, G:2 * G], kv)
    np.testing.assert_array_equal(y, native.attend_online(qr[0, G:2 * G], host.view(1).select(slice(0, 5)), f)[0])


def test_device_view_reads_as_the_references_compressed_kv(ctx):
    """DeviceKV's arrays are the decoded device rows (the oracle's CompressedKV on
    the same rows); a selection that is not a prefix is a host CompressedKV."""
    from insitu_amd import QuantConfig
    from insitu_amd.cache import CompressedCache, CompressedKV
    rng = np.random.default_rng(9)
    f = Format()
    T = 30
    k = rng.integers(-(1 << 22), 1 << 22, size=(T, 8, 64))
    v = rng.integers(-(1 << 22), 1 << 22, size=(T, 8, 64))
    cache = CompressedCache(8, 64, T, QuantConfig(key_bits=4, value_bits=2), ctx=ctx)
    cache.append_rotated(k, v)
    host = Cache(8, T, f)
    host.append_rotated(k, v)
    for h in (0, 7):
        got, want = cache.view(h), host.view(h)
        for name in ("k_idx", "k_norm", "v_idx", "v_norm"):
            np.testing.assert_array_equal(getattr(got, name), getattr(want, name), err_msg=name)
        part = got.select(slice(3, 20, 2))
        assert isinstance(part, CompressedKV)
        np.testing.assert_array_equal(part.k_idx, want.k_idx[3:20:2])
        assert got.select(slice(0, -4)).n_tokens == T - 4
