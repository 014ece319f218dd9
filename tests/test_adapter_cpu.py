"""The adapter's host-side pieces, on the CPU (tests/test_adapter.py:46-49 of the
reference): the model shape read from a transformers-style config, and the adapter
module importing without a GPU."""

from insitu_amd import ModelConfig


class _StubConfig:
    hidden_size = 128
    num_attention_heads = 4
    num_key_value_heads = 2
    head_dim = 32
    rope_theta = 10000.0
    max_position_embeddings = 256


def test_model_config_from_hf():
    m = ModelConfig.from_hf(_StubConfig)
    assert (m.hidden_size, m.num_heads, m.num_kv_heads, m.head_dim) == (128, 4, 2, 32)
    assert m.kv_groups == 2


def test_model_config_from_a_transformers_llama_config():
    from transformers import LlamaConfig
    c = LlamaConfig(hidden_size=2048, num_attention_heads=32, num_key_value_heads=8, head_dim=64,
                    rope_theta=500000.0, max_position_embeddings=131072,
                    rope_scaling={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
                                  "high_freq_factor": 4.0, "original_max_position_embeddings": 8192})
    m = ModelConfig.from_hf(c)
    assert (m.num_heads, m.num_kv_heads, m.head_dim, m.kv_groups) == (32, 8, 64, 4)
    assert m.rope_theta == 500000.0 and m.max_position == 131072
    assert m.rope_scaling is not None and m.rope_scaling.factor == 32.0


def test_adapter_module_imports_without_a_gpu():
    from insitu_amd.adapters import torch_llama
    for name in ("KernelAttention", "build_from_layer", "graft", "ungraft", "compare_against_original"):
        assert callable(getattr(torch_llama, name))
