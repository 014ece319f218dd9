"""The chunked attend's two builds: 1,024-token chunks (the default of a bare cache) and
512-token chunks (the default of AttentionBlock, for a model's flat softmax).

The attend tests of test_gpu_parity that make their caches with `_cache` run again here
on 512-token chunks, and the fused-step tests that make an AttentionBlock run again on
1,024-token chunks, so that both builds meet the same oracle checks.
"""

import functools

import numpy as np
import pytest

import test_gpu_parity as P

pytestmark = pytest.mark.gpu


@pytest.fixture
def chunk512(monkeypatch):
    monkeypatch.setattr(P, "_cache", functools.partial(P._cache, chunk_tokens=512))


@pytest.fixture
def blocks1024(monkeypatch):
    import insitu_amd.block as block

    base = block.AttentionBlock

    class Block1024(base):
        def __init__(self, *a, **kw):
            kw["chunk_tokens"] = 1024
            super().__init__(*a, **kw)

    monkeypatch.setattr(block, "AttentionBlock", Block1024)


@pytest.mark.parametrize("mode", ["online", "two_pass"])
@pytest.mark.parametrize("T", [63, 511, 512, 513, 700, 3000])
def test_random_contexts_on_512_token_chunks(ctx, chunk512, mode, T):
    P.test_attend_random_contexts_against_native_oracle(ctx, mode, T)


def test_full_c2_context_on_512_token_chunks(ctx, chunk512):
    P.test_full_c2_context_against_native_oracle(ctx, "online")


def test_ragged_batch_on_512_token_chunks(ctx, chunk512):
    P.test_ragged_batch_multi_chunk(ctx)


@pytest.mark.parametrize("mode", ["online", "two_pass"])
def test_many_chains_on_512_token_chunks(ctx, chunk512, mode):
    P.test_many_chains_merge_their_statistics(ctx, mode)


def test_run_pool_fallback_on_512_token_chunks(ctx, chunk512):
    P.test_rising_scores_exhaust_the_run_pool_and_fall_back_exactly(ctx)


def test_later_chunk_replay_on_512_token_chunks(ctx, chunk512):
    P.test_a_later_chunk_replays_from_chunk_zeros_published_state(ctx)


@pytest.mark.parametrize("mode", ["online", "two_pass"])
def test_prefill_on_512_token_chunks(ctx, chunk512, mode):
    P.test_prefill_from_a_base_across_chunks_and_query_batches(ctx, mode)


@pytest.mark.parametrize("mode", ["online", "two_pass", "serial"])
@pytest.mark.parametrize("d,kb,vb", [(64, 4, 2), (128, 3, 3)])
def test_fused_step_on_1024_token_chunks(ctx, blocks1024, mode, d, kb, vb):
    P.test_fused_step_ragged_batch_multi_chunk(ctx, mode, d, kb, vb)


def test_flat_softmax_on_1024_token_chunks(ctx, blocks1024):
    P.test_fused_step_over_a_flat_softmax(ctx)


@pytest.mark.parametrize("softmax", ["online", "two_pass"])
def test_block_prefill_on_1024_token_chunks(ctx, blocks1024, softmax):
    P.test_block_prefill_equals_the_decode_loop(ctx, softmax)


def test_the_online_block_uses_512_token_chunks_two_pass_and_a_bare_cache_1024(ctx):
    from insitu_amd import ModelConfig, QuantConfig
    from insitu_amd.block import AttentionBlock
    blk = AttentionBlock(ModelConfig.llama32_1b(), QuantConfig(key_bits=4, value_bits=2),
                         capacity=600, ctx=ctx)
    assert blk.cache.chunk_tokens == 512
    two = AttentionBlock(ModelConfig.llama32_1b(), QuantConfig(key_bits=4, value_bits=2),
                         capacity=600, softmax="two_pass", ctx=ctx)
    assert two.cache.chunk_tokens == 1024
    assert P._cache(ctx, 600).chunk_tokens == 0


@pytest.mark.parametrize("mode", ["online", "two_pass"])
def test_static_prefill_on_512_token_chunks(ctx, monkeypatch, mode):
    """The allocation-free prefill lays its static array out by the cache's build."""
    import test_zz_no_alloc as Z
    monkeypatch.setattr(Z, "_cache", functools.partial(Z._cache, chunk_tokens=512))
    Z.test_static_prefill_equals_the_allocating_prefill_twice(ctx, mode)


@pytest.mark.parametrize("bad", [256, 1023, 2048, -1])
def test_other_chunk_sizes_are_refused(ctx, bad):
    from insitu_amd._lib import InsituError
    with pytest.raises(InsituError, match="chunk_tokens"):
        P._cache(ctx, 600, chunk_tokens=bad)
