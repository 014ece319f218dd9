"""The configuration the seam half needs: QuantConfig, FixedFormat, ModelConfig.

Same names, fields, defaults and validation as config.py:33-254 of the
reference, restricted to what the compressed-KV decode path reads. Note the
reference's trap, kept on purpose: `QuantConfig()` defaults to 3-bit keys
while the reference's goldens and board are 4-bit (config.py:141).
"""

from __future__ import annotations

import math
from dataclasses import dataclass


@dataclass(frozen=True)
class ModelConfig:
    """config.py:33-76: the attention shape, and the RoPE settings the host half uses."""

    hidden_size: int
    num_heads: int
    num_kv_heads: int
    head_dim: int | None = None
    rope_theta: float = 10000.0
    max_position: int = 4096
    rope_scaling: object | None = None     # insitu_amd.host.RopeScaling, or None for plain RoPE

    def __post_init__(self) -> None:
        d = self.head_dim if self.head_dim is not None else self.hidden_size // self.num_heads
        object.__setattr__(self, "head_dim", d)
        if self.num_heads % self.num_kv_heads:
            raise ValueError(f"num_heads={self.num_heads} must be a multiple of "
                             f"num_kv_heads={self.num_kv_heads} (grouped-query attention)")
        if d & (d - 1):
            raise ValueError(f"head_dim={d} must be a power of two: the rotation is a "
                             f"Walsh-Hadamard butterfly")
        if d % 2:
            raise ValueError(f"head_dim={d} must be even")

    @property
    def kv_groups(self) -> int:
        return self.num_heads // self.num_kv_heads

    @property
    def q_out_features(self) -> int:
        return self.num_heads * self.head_dim

    @property
    def kv_out_features(self) -> int:
        return self.num_kv_heads * self.head_dim

    @classmethod
    def from_hf(cls, hf_config) -> "ModelConfig":
        """config.py:78-120: from a transformers config (or anything duck-typed, a
        dict included). rope_theta is read top-level or from rope_parameters and
        never defaulted; "default" and "llama3" RoPE are modelled, any other
        scaling type is refused."""
        from .host import RopeScaling
        get = (lambda k, d=None: hf_config.get(k, d)) if isinstance(hf_config, dict) \
            else (lambda k, d=None: getattr(hf_config, k, d))
        theta = get("rope_theta")
        params = get("rope_parameters") or {}
        if theta is None:
            theta = params.get("rope_theta")
        if theta is None:
            raise ValueError("config exposes neither `rope_theta` nor `rope_parameters['rope_theta']`; "
                             "pass ModelConfig directly rather than defaulting a value that decides "
                             "token positions")
        if not params and isinstance(get("rope_scaling"), dict):
            params = get("rope_scaling")
        rope_type = params.get("rope_type") or params.get("type") or "default"
        if rope_type == "llama3":
            scaling = RopeScaling.from_hf(params)
        elif rope_type == "default":
            scaling = None
        else:
            raise NotImplementedError(f"RoPE scaling {rope_type!r} is not modelled")
        return cls(hidden_size=get("hidden_size"), num_heads=get("num_attention_heads"),
                   num_kv_heads=get("num_key_value_heads", get("num_attention_heads")),
                   head_dim=get("head_dim"), rope_theta=float(theta),
                   max_position=get("max_position_embeddings", 4096), rope_scaling=scaling)

    @classmethod
    def tinyllama(cls) -> "ModelConfig":
        """config.py:122-125: TinyLlama-1.1B."""
        return cls(hidden_size=2048, num_heads=32, num_kv_heads=4, head_dim=64)

    @classmethod
    def llama32_1b(cls) -> "ModelConfig":
        """Llama-3.2-1B attention shape (hw/vectors.py:831)."""
        return cls(hidden_size=2048, num_heads=32, num_kv_heads=8, head_dim=64)

    @classmethod
    def llama3_8b(cls) -> "ModelConfig":
        return cls(hidden_size=4096, num_heads=32, num_kv_heads=8, head_dim=128)


@dataclass(frozen=True)
class QuantConfig:
    """config.py:132-207."""

    key_bits: int = 3
    value_bits: int = 2
    norm_bits: int = 16
    norm_frac: int = 9
    seed: int = 0
    symmetric: bool = True
    rot_rounds: int = 1
    codebook: str = "gaussian"

    def __post_init__(self) -> None:
        for name, b in (("key_bits", self.key_bits), ("value_bits", self.value_bits)):
            if not 1 <= b <= 8:
                raise ValueError(f"{name}={b} outside the supported range 1..8")
        if self.rot_rounds < 0:
            raise ValueError(f"rot_rounds={self.rot_rounds} must not be negative")
        if self.codebook not in ("gaussian", "uniform"):
            raise ValueError(f"codebook={self.codebook!r}; expected gaussian or uniform")
        if self.norm_frac >= self.norm_bits:
            raise ValueError(f"norm_frac={self.norm_frac} leaves no integer bits in "
                             f"norm_bits={self.norm_bits}")

    def bytes_per_token(self, head_dim: int) -> int:
        """config.py:192-207: one compressed token of one KV head."""
        code_bits = head_dim * (self.key_bits + self.value_bits)
        if code_bits % 8:
            raise ValueError(f"head_dim*(key_bits+value_bits) = {code_bits} is not a whole "
                             f"number of bytes; choose widths summing to a multiple of "
                             f"{8 // math.gcd(8, head_dim)}")
        return code_bits // 8 + 2 * (self.norm_bits // 8)


@dataclass(frozen=True)
class FixedFormat:
    """config.py:214-254."""

    qk_frac: int = 16
    qk_width: int = 24
    centroid_frac: int = 15
    acc_frac: int = 16
    acc_width: int = 32
    score_width: int = 48
    prob_frac: int = 15
    prob_width: int = 16
    exp_lut_bits: int = 8
    saturate: bool = True
    recip_norm_bits: int = 32

    def score_shift_for(self, quant: QuantConfig) -> int:
        return self.qk_frac + self.centroid_frac + quant.norm_frac - self.acc_frac

    def acc_shift_for(self, quant: QuantConfig) -> int:
        return self.centroid_frac + quant.norm_frac + self.prob_frac - self.acc_frac
