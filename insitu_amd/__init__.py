"""insitu_amd: the compressed-KV decode-attention block of INSITU on MI355X (gfx950).

The seam half of the reference's AttentionKernel (rotate -> quantize + append
-> score on codes -> fixed-point online softmax -> Q16 out) as hand-written
HIP kernels in libinsitu_hip.so, behind a C ABI (include/insitu.h), with a
Python host side that mirrors the reference's interfaces:

    QuantConfig, FixedFormat, ModelConfig   config.py of the reference
    Codebook                                ops/codebook.py
    Rotation                                ops/rotate.py
    KVCache, CompressedCache                cache/base.py, cache/compressed.py
    CompressedAttention, AttentionStats     ops/attention.py
    AttentionBlock, StepReport              kernel.py (forward, both halves)
    Weights, HostHalf, RoPE, RopeScaling    weights.py, ops/rope.py, kernel.py:198-249
"""

from .config import FixedFormat, ModelConfig, QuantConfig
from .codebook import Codebook

__all__ = ["FixedFormat", "ModelConfig", "QuantConfig", "Codebook", "Rotation",
           "KVCache", "CompressedCache", "CompressedKV", "CompressedAttention",
           "AttentionStats", "AttentionBlock", "StepReport", "Weights", "HostHalf", "RoPE",
           "RopeScaling"]


def __getattr__(name):
    # The device-facing classes import lazily so `import insitu_amd` works on a
    # machine without a GPU (the build check); using them still needs the library.
    if name == "Rotation":
        from .rotate import Rotation
        return Rotation
    if name in ("KVCache", "CompressedCache", "CompressedKV"):
        from . import cache
        return getattr(cache, name)
    if name in ("CompressedAttention", "AttentionStats"):
        from . import attention
        return getattr(attention, name)
    if name in ("AttentionBlock", "StepReport"):
        from . import block
        return getattr(block, name)
    if name in ("Weights", "HostHalf", "RoPE", "RopeScaling"):
        from . import host
        return getattr(host, name)
    raise AttributeError(name)
