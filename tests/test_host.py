"""Host-side logic of the product, and the C ABI's surface, without a GPU."""

import ctypes
import os
import re

import numpy as np
import pytest

from oracle import hexio as hx
from oracle.codebook import gaussian
from oracle.quantize import CompressedKV, Format, pack

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_product_codebooks_match_the_goldens_and_the_oracle():
    from insitu_amd.codebook import Codebook
    np.testing.assert_array_equal(Codebook.gaussian(4).centroids, hx.scalars("cb_centroids_key.hex", 20))
    np.testing.assert_array_equal(Codebook.gaussian(4).boundaries, hx.scalars("enc_bounds_key.hex", 20))
    np.testing.assert_array_equal(Codebook.gaussian(2).centroids, hx.scalars("cb_centroids_value.hex", 20))
    np.testing.assert_array_equal(Codebook.gaussian(2).boundaries, hx.scalars("enc_bounds_value.hex", 20))
    for bits in range(1, 9):
        c, b = gaussian(bits)
        np.testing.assert_array_equal(Codebook.gaussian(bits).centroids, c)
        np.testing.assert_array_equal(Codebook.gaussian(bits).boundaries, b)
    u = Codebook.uniform(3)
    assert np.all(np.diff(u.centroids) > 0)
    with pytest.raises(ValueError):
        Codebook.build("nope", 2)


def test_product_rotation_signs():
    from insitu_amd.rotate import Rotation
    assert Rotation.from_seed(64, 0).sign_words() == [(0x81191FF5899001F8, 0)]
    r = Rotation.from_seed(128, 0)
    w0, w1 = r.sign_words()[0]
    for i in range(128):
        bit = ((w0 if i < 64 else w1) >> (i % 64)) & 1
        assert bit == int(r.signs[0, i] < 0)
    with pytest.raises(ValueError):
        Rotation.from_seed(48, 0)


def test_product_unpack_rows_matches_the_oracle_format():
    from insitu_amd.cache import unpack_rows
    rows = hx.bytes_rows("cache_rows_h3.hex")
    kv = unpack_rows(rows, 64, 4, 2)
    back = pack(CompressedKV(kv.k_idx, kv.k_norm, kv.v_idx, kv.v_norm), Format())
    np.testing.assert_array_equal(back, rows)
    rng = np.random.default_rng(0)
    f = Format(d=128, key_bits=3, value_bits=3)
    kv = CompressedKV(rng.integers(0, 8, (5, 128)).astype(np.uint8), np.array([1, -1, 7, -32768, 32767]),
                      rng.integers(0, 8, (5, 128)).astype(np.uint8), np.array([0, 2, -3, 4, 5]))
    got = unpack_rows(pack(kv, f), 128, 3, 3)
    np.testing.assert_array_equal(got.k_idx, kv.k_idx)
    np.testing.assert_array_equal(got.v_norm, kv.v_norm)


def test_config_validation_mirrors_the_reference():
    from insitu_amd.config import FixedFormat, ModelConfig, QuantConfig
    assert QuantConfig().key_bits == 3                  # the reference's default (config.py:141)
    assert QuantConfig(key_bits=4).bytes_per_token(64) == 52
    assert QuantConfig(key_bits=3, value_bits=3).bytes_per_token(128) == 100
    with pytest.raises(ValueError):
        QuantConfig(key_bits=9)
    with pytest.raises(ValueError):
        QuantConfig(norm_frac=16)
    with pytest.raises(ValueError):
        ModelConfig(hidden_size=2048, num_heads=32, num_kv_heads=7, head_dim=64)
    with pytest.raises(ValueError):
        ModelConfig(hidden_size=2048, num_heads=32, num_kv_heads=8, head_dim=48)
    assert ModelConfig.llama32_1b().kv_groups == 4
    f = FixedFormat()
    assert f.score_shift_for(QuantConfig()) == 24 and f.acc_shift_for(QuantConfig()) == 23


def test_workload_generator_is_deterministic_and_in_range():
    from insitu_amd.workload import Workload, to_fixed
    a = Workload(seed=0).steps(3)
    b = Workload(seed=0).steps(3)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)
    q, k, v = a
    assert q.shape == (1, 3, 32, 64) and k.shape == (1, 3, 8, 64)
    assert np.abs(q).max() < (1 << 23)
    np.testing.assert_array_equal(to_fixed([0.5 / 65536, 1.5 / 65536, 1e6, -1e6]),
                                  [0, 2, (1 << 23) - 1, -(1 << 23)])
    w = Workload(seed=1, head_dim=128, outlier_mode="percent")
    assert w.q_scale.shape == (32, 128) and set(np.unique(w.q_scale)) <= {1.0, 16.0}


def test_library_exports_every_declared_symbol():
    """The C ABI loads and exports exactly what include/insitu.h declares (no GPU call)."""
    from insitu_amd import _lib
    hdr = open(os.path.join(ROOT, "include", "insitu.h")).read()
    declared = set(re.findall(r"\b(insitu_[a-z_]+)\s*\(", hdr))
    assert declared == set(_lib.EXPORTS), declared ^ set(_lib.EXPORTS)
    if not os.path.exists(_lib.LIB_PATH):
        from insitu_amd.build import build
        build()
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in sorted(declared):
        assert hasattr(lib, name), name
    loaded = _lib.load()
    assert loaded.insitu_last_error() is not None


def test_product_never_imports_the_oracle():
    pkg = os.path.join(ROOT, "insitu_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"^\s*(from|import)\s+oracle\b", text, re.M), f
                assert "liboracle" not in text, f


def test_fp64_quotient_method_of_the_device_reciprocal():
    """The kernels compute floor(2^62 / n), n in [2^31, 2^48), as the correctly
    rounded fp64 quotient truncated, minus one when r * n > 2^62. Checked here
    against exact integer division, numpy's float64 division being IEEE like the
    GPU's, on random n and on n whose quotient sits just below an integer."""
    rng = np.random.default_rng(11)
    n = np.concatenate([
        rng.integers(1 << 31, 1 << 32, size=200_000),
        rng.integers(1 << 32, 1 << 48, size=200_000),
        [1 << 31, (1 << 32) - 1, (1 << 47) + 1, (1 << 48) - 1],
    ]).astype(np.uint64)
    q = (np.uint64(1) << np.uint64(62)) // n
    near = (np.uint64(1) << np.uint64(62)) // (q + np.uint64(1)) + np.uint64(1)
    n = np.concatenate([n, near[(near >= (1 << 31)) & (near < (1 << 48))]])
    exact = (np.uint64(1) << np.uint64(62)) // n
    r = (4611686018427387904.0 / n.astype(np.float64)).astype(np.uint64)
    r = np.where(r * n > (np.uint64(1) << np.uint64(62)), r - np.uint64(1), r)
    np.testing.assert_array_equal(r, exact)


def test_host_half_tables_and_fold_match_the_oracle():
    """insitu_amd.host builds the RoPE tables and the W_o fold on the host; the
    oracle's restatements (pinned to the reference's goldens) give the same."""
    from insitu_amd.host import RoPE, RopeScaling, fold_o_proj
    from oracle import host as oh
    from oracle.rotate import matrix, signs_from_seed
    for theta, scaling in ((10000.0, None), (500000.0, (32.0, 1.0, 4.0, 8192))):
        t = RoPE.build(64, 3000, theta, scaling=RopeScaling(*scaling) if scaling else None)
        cos, sin = oh.rope_tables(64, 3000, theta, scaling=oh.RopeScaling(*scaling) if scaling else None)
        np.testing.assert_array_equal(t.cos, cos)
        np.testing.assert_array_equal(t.sin, sin)
    hf = RopeScaling.from_hf({"factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                              "original_max_position_embeddings": 8192, "rope_type": "llama3"})
    assert hf == RopeScaling(32.0, 1.0, 4.0, 8192)
    with pytest.raises(ValueError):
        RopeScaling(8.0, 4.0, 1.0, 8192)
    with pytest.raises(ValueError):
        RoPE.build(63, 8)
    sg = signs_from_seed(64, 0, 1)
    wo = np.random.default_rng(2).standard_normal((32, 3 * 64))
    np.testing.assert_allclose(fold_o_proj(wo, matrix(sg), 3), oh.fold_o_proj(wo, sg, 3), rtol=0, atol=1e-12)
    with pytest.raises(ValueError):
        fold_o_proj(wo, matrix(sg), 2)


def _ddr_fixture():
    import json
    from insitu_amd.interop import DdrLayout
    with open(os.path.join(ROOT, "tests", "golden", "tb_vectors", "ddr_map.json")) as f:
        d = json.load(f)
    lay = DdrLayout.from_describe(d, ((0, 32), (32, 48), (48, 52)))
    rows = np.stack([hx.bytes_rows(f"cache_rows_h{h}.hex") for h in range(8)], axis=1)
    return d, lay, rows


def test_interop_layout_builds_the_golden_ddr_image_and_inverts_it():
    """hw/ddr_layout.py:227-274: the product's address map against ddr_map.json and
    ddr_image.hex; rows() and row_at() invert image()."""
    d, lay, rows = _ddr_fixture()
    assert lay.describe() == d
    img = lay.image(rows)
    np.testing.assert_array_equal(img, hx.bytes_rows("ddr_image.hex").reshape(-1))
    np.testing.assert_array_equal(lay.rows(img, 65), rows)
    for h, t in ((0, 0), (7, 64), (3, 31)):
        np.testing.assert_array_equal(lay.row_at(img, h, t), rows[t, h])
    with pytest.raises(ValueError):
        lay.image(rows[:, :7])
    with pytest.raises(ValueError):
        lay.rows(img[:100], 65)


def test_cache_diff_names_the_field_of_every_differing_row():
    """experiments/cache_diff.py:91-121: a planted byte in each field is reported
    at its (head, token) with the field it lies in; equal caches match."""
    from insitu_amd.interop import cache_diff
    _, lay, rows = _ddr_fixture()
    assert cache_diff(rows, rows.copy(), lay.fields).match
    bad = rows.copy()
    bad[5, 2, 3] ^= 0x10          # key codes
    bad[64, 7, 40] ^= 1           # value codes
    bad[0, 0, 50] ^= 0x80         # norms
    bad[9, 4, [0, 33]] ^= 1       # key and value
    rep = cache_diff(bad, rows, lay.fields)
    got = [(r.head, r.token, r.fields, r.n_bytes) for r in rep.rows]
    assert got == [(0, 0, ["norms"], 1), (2, 5, ["key"], 1), (4, 9, ["key", "value"], 2),
                   (7, 64, ["value"], 1)]
    assert "key+value+norms" in rep.verdict()
    with pytest.raises(ValueError):
        cache_diff(bad[:3], rows, lay.fields)


def test_product_rotation_matrix_is_the_oracles():
    from insitu_amd.rotate import Rotation
    from oracle.rotate import matrix, signs_from_seed
    for d, rounds in ((64, 1), (128, 2)):
        r = Rotation.from_seed(d, 0, rounds)
        np.testing.assert_array_equal(r.matrix(), matrix(signs_from_seed(d, 0, rounds)))
        np.testing.assert_allclose(r.matrix() @ r.matrix().T, np.eye(d), atol=1e-12)


def test_model_config_from_hf_reads_rope_settings_or_refuses():
    """config.py:78-120: theta top-level or nested, llama3 scaling modelled, other
    scaling types refused, a missing theta refused rather than defaulted."""
    from insitu_amd import ModelConfig
    from insitu_amd.host import RopeScaling
    llama = {"hidden_size": 2048, "num_attention_heads": 32, "num_key_value_heads": 8, "head_dim": 64,
             "rope_theta": 500000.0, "max_position_embeddings": 131072,
             "rope_scaling": {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
                              "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}}
    m = ModelConfig.from_hf(llama)
    assert (m.num_kv_heads, m.head_dim, m.max_position, m.rope_theta) == (8, 64, 131072, 500000.0)
    assert m.rope_scaling == RopeScaling(32.0, 1.0, 4.0, 8192)
    nested = {k: v for k, v in llama.items() if k not in ("rope_theta", "rope_scaling")}
    nested["rope_parameters"] = {"rope_theta": 1e4, "rope_type": "default"}
    m = ModelConfig.from_hf(nested)
    assert m.rope_theta == 1e4 and m.rope_scaling is None
    with pytest.raises(ValueError):
        ModelConfig.from_hf({k: v for k, v in nested.items() if k != "rope_parameters"})
    with pytest.raises(NotImplementedError):
        ModelConfig.from_hf(dict(llama, rope_scaling={"rope_type": "yarn", "factor": 4.0}))


def test_checkpoint_tensors_convert_for_the_weights():
    import torch
    from insitu_amd.host import _host_array
    w = torch.randn(4, 3, requires_grad=True).half()
    got = _host_array(w)
    assert got.dtype == np.float32 and got.shape == (4, 3)
    np.testing.assert_array_equal(got.astype(np.float16), w.detach().numpy())
    assert _host_array(None) is None


def _layout(lib, kernel, capacity, batch=1, n_kv=8, d=64):
    f = (ctypes.c_int64 * 11)()
    rc = lib.insitu_debug_scratch_layout(kernel, capacity, batch, n_kv, d, f, 11)
    assert rc == 0, lib.insitu_last_error()
    return dict(zip(["chunks", "pool", "slots", "last_end", "nseg", "hmax", "bytes", "front", "areas_ok",
                     "chunk_tokens", "slot_limit"], list(f)))


@pytest.mark.parametrize("kernel", [0, 1, 2])
def test_scratch_layout_invariants(kernel):
    """The replay's indices stay inside the carve (computed on the host, no GPU call): every
    chunk's run slots fit the pool with the spare slot after them, slot ids fit 15 bits, the
    areas are aligned and disjoint, and the epoch-checked front comes first."""
    from insitu_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    lib = _lib.load()
    for d in ([64, 128] if kernel < 2 else [64]):
        for batch in (1, 3):
            for cap in (1, 1023, 1024, 1025, 32768, 262144, 300000, 524288):
                f = _layout(lib, kernel, cap, batch, 8, d)
                assert f["chunks"] == -(-cap // f["chunk_tokens"])
                if f["chunks"] > f["hmax"]:
                    continue                  # a capacity the kernel refuses
                assert f["areas_ok"] == 1, f
                # the last chunk's slots end at pool - 1: the spare slot is never written
                assert f["last_end"] == f["pool"] - 1, f
                assert f["pool"] < f["slot_limit"], f
                assert 0 < f["front"] <= f["bytes"], f
    # The replay lists at most NSEG runs per head, fewer than the most a sequence can publish
    # (HMAX - 1 chunks x SLOTS): the list's length is checked before the walk, and a head past
    # it takes the serial path.
    f = _layout(lib, kernel, 1024 * 512)
    assert f["nseg"] < (f["hmax"] - 1) * f["slots"]
    src = open(os.path.join(ROOT, "insitu_amd", "csrc",
                            "attend_step.hip" if kernel == 2 else "attend_chunked.hip")).read()
    assert "total > NSEG" in src


def test_block_chunk_size_follows_capacity():
    """A block's cache takes 512-token chunks only while the chunked attend's chunk limit
    holds them; past 262,144 tokens it keeps 1,024-token chunks (and the chunked path)."""
    from insitu_amd import _lib
    from insitu_amd.block import CHUNKED_MAX_CHUNKS, default_chunk_tokens
    src = open(os.path.join(ROOT, "insitu_amd", "csrc", "attend_chunked.hip")).read()
    assert re.search(r"constexpr int HMAX = (\d+);", src).group(1) == str(CHUNKED_MAX_CHUNKS)
    assert default_chunk_tokens("online", 262144) == 512
    assert default_chunk_tokens("online", 300000) == 1024
    assert default_chunk_tokens("split", 300000) == 1024
    assert default_chunk_tokens("two_pass", 1000) == 1024
    if os.path.exists(_lib.LIB_PATH):
        lib = _lib.load()
        for cap in (262144, 300000, 524288):
            kernel = 1 if default_chunk_tokens("online", cap) == 512 else 0
            f = _layout(lib, kernel, cap)
            assert f["chunks"] <= f["hmax"], (cap, f)
