"""GPU: the vectors tests/golden/make_reference_vectors.py wrote from the reference itself,
reproduced on the device bit for bit.

  d128_3b3b_ctx64.npz   Llama-3-8B attention shape (d = 128, 3-bit keys and values):
                        the cache's 64 context rows are loaded (CMD_LOAD), then one
                        insitu_step from the wire rows; the codebooks, the appended row
                        and the Q16 output in both softmax modes equal the reference's.
  d64_4b2b_ctx512.npz   the same at config 0's context (512 + 1).
  d64_4b2b_steps_from_empty.npz
                        40 insitu_steps from an empty cache: every appended row and
                        every step's online output.
"""

import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def _block(ctx, d, kb, vb, capacity, softmax):
    from insitu_amd import ModelConfig, QuantConfig
    from insitu_amd.block import AttentionBlock
    model = ModelConfig(hidden_size=32 * d, num_heads=32, num_kv_heads=8, head_dim=d)
    return AttentionBlock(model, QuantConfig(key_bits=kb, value_bits=vb), capacity=capacity,
                          softmax=softmax, ctx=ctx)


@pytest.mark.parametrize("name,d,kb,vb", [("d128_3b3b_ctx64.npz", 128, 3, 3),
                                          ("d64_4b2b_ctx512.npz", 64, 4, 2)],
                         ids=["d128_3b3b", "d64_4b2b_ctx512"])
@pytest.mark.parametrize("softmax", ["online", "two_pass", "serial"])
def test_one_step_over_the_loaded_context(ctx, name, d, kb, vb, softmax):
    z = _load(name)
    n = int(z["context"])
    blk = _block(ctx, d, kb, vb, n + 1, softmax)
    c = blk.cache
    np.testing.assert_array_equal(c.key_codebook.centroids, z["key_centroids"])
    np.testing.assert_array_equal(c.key_codebook.boundaries, z["key_bounds"])
    np.testing.assert_array_equal(c.value_codebook.centroids, z["value_centroids"])
    np.testing.assert_array_equal(c.value_codebook.boundaries, z["value_bounds"])
    for h in range(8):
        c.load_rows(z["cache"][:n, h], h)
    c.set_length(n)
    out = blk.step(z["wire_q"], z["wire_k"], z["wire_v"]).cpu().numpy()
    want = z["out_two_pass"] if softmax == "two_pass" else z["out_online"]
    np.testing.assert_array_equal(out, want)
    for h in range(8):
        np.testing.assert_array_equal(c.read_rows(h, n, 1)[0], z["row"][h], err_msg=f"row of KV head {h}")
    assert c.length == n + 1


def test_forty_steps_from_an_empty_cache(ctx):
    z = _load("d64_4b2b_steps_from_empty.npz")
    steps = z["wire_q"].shape[0]
    blk = _block(ctx, 64, 4, 2, steps, "online")
    for t in range(steps):
        out = blk.step(z["wire_q"][t][None], z["wire_k"][t][None], z["wire_v"][t][None]).cpu().numpy()
        np.testing.assert_array_equal(out[0], z["out_online"][t], err_msg=f"step {t}")
    for h in range(8):
        np.testing.assert_array_equal(blk.cache.read_rows(h, 0, steps), z["rows"][:, h], err_msg=f"KV head {h}")
