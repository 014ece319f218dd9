"""The GPU attention block in place of a Llama-family model's attention module.

    from insitu_amd.adapters.torch_llama import graft

    model = AutoModelForCausalLM.from_pretrained(...)
    graft(model, layers=[10], quant=QuantConfig(key_bits=3, value_bits=2))

The names, arguments and behaviour are those of adapters/torch_llama.py of the
reference (KernelAttention, build_from_layer, graft, ungraft,
compare_against_original), with AttentionBlock (the whole block on the GPU:
fp16 projections, scale, RoPE and the cast to the wire, then rotate, append,
attend on the codes and W_o') in place of the numpy AttentionKernel. The
hidden states stay on the device; nothing crosses to numpy on the way.

The contract a decoder layer calls (transformers' LlamaAttention) is kept as
the reference keeps it:

  * `position_ids` give the tokens' positions (`cache_position` is the older
    spelling); without either the block counts from its own cache length.
  * `past_key_values` is advanced with zero K/V of the right shape, so the
    model's own length bookkeeping stays right; it is never read back: the
    compressed cache is the block's own.
  * `attention_mask` and `position_embeddings` are ignored: the block is causal
    by construction and applies RoPE itself. A batch of more than one sequence
    is refused rather than attended across.

Differences from the reference, by construction: the host half runs its fp32
GEMVs on the GPU, so a wire row can differ from the reference's numpy float
order by up to 2 Q8.16 LSB in a few lanes (below the seam everything is
bit-exact for the same wire rows); QK-norm models, the dense fp16 baseline
(compressed=False) and the reference's hardware model (hw) are refused with
NotImplementedError rather than approximated.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn as nn

from ..block import AttentionBlock
from ..config import FixedFormat, ModelConfig, QuantConfig
from ..host import Weights


class KernelAttention(nn.Module):
    """torch_llama.py:58-155: a module with the shape of a Llama attention module,
    holding an AttentionBlock."""

    def __init__(self, kernel: AttentionBlock, layer_idx: int = 0, dtype=None, device=None) -> None:
        super().__init__()
        self.kernel = kernel
        self.layer_idx = layer_idx
        self._dtype = dtype
        self._device = device
        self.last_report = None

    def forward(self, hidden_states, *args, **kwargs):
        """(batch, seq, hidden) or (seq, hidden) in, (output of the same shape, None) out."""
        x = hidden_states
        squeeze = x.dim() == 2
        if squeeze:
            x = x.unsqueeze(0)
        if x.shape[0] != 1:
            raise NotImplementedError(
                f"batch of {x.shape[0]}: this adapter holds one sequence's cache and ignores "
                f"attention_mask, so a padded batch would silently attend across sequences. "
                f"Run one sequence at a time.")
        positions = kwargs.get("position_ids")
        if positions is None:
            positions = kwargs.get("cache_position")
        pos = None
        if positions is not None:
            pos = positions.reshape(-1).detach().cpu().numpy().astype(np.int64)
        y, report = self.kernel.forward(x[0].detach(), pos)
        self.last_report = report
        self._advance_hf_cache(kwargs.get("past_key_values"), x)
        out = y.to(device=x.device, dtype=self._dtype or hidden_states.dtype)
        return (out if squeeze else out.unsqueeze(0)), None

    def _advance_hf_cache(self, cache, x) -> None:
        """torch_llama.py:137-159: bookkeeping only, so that
        past_key_values.get_seq_length() stays the truth."""
        if cache is None:
            return
        m = self.kernel.model
        filler = torch.zeros((x.shape[0], m.num_kv_heads, x.shape[1], m.head_dim),
                             dtype=x.dtype, device=x.device)
        try:
            cache.update(filler, filler, self.layer_idx)
        except Exception as e:
            raise RuntimeError(
                f"could not advance past_key_values ({type(cache).__name__}) for layer "
                f"{self.layer_idx}; positions after the first token would be wrong. Pass "
                f"past_key_values=None, or update this shim.") from e

    def reset(self) -> None:
        self.kernel.reset()


def build_from_layer(attn_module, model_config, *, quant: QuantConfig | None = None,
                     fmt: FixedFormat | None = None, hw=None, capacity: int = 4096,
                     compressed: bool = True, layer_idx: int = 0, softmax: str = "two_pass",
                     ctx=None) -> KernelAttention:
    """torch_llama.py:172-203: a KernelAttention from an attention module's weights.

    softmax defaults to the reference AttentionKernel's default, "two_pass";
    "online" is the hardware's order and the single fused launch per decode step.
    """
    if not compressed:
        raise NotImplementedError("compressed=False is the reference's fp16 dense baseline; "
                                  "this build runs the compressed block only")
    if hw is not None:
        raise NotImplementedError("hw configures the reference's systolic-array model; the GPU "
                                  "block has no counterpart")
    if getattr(attn_module, "q_norm", None) is not None or getattr(attn_module, "k_norm", None) is not None:
        raise NotImplementedError("QK-norm (q_norm / k_norm) is not modelled by the GPU host half")
    m = ModelConfig.from_hf(model_config)
    block = AttentionBlock(m, quant or QuantConfig(), fmt, capacity=capacity, softmax=softmax, ctx=ctx)

    def w(name):
        return getattr(attn_module, f"{name}_proj").weight

    def b(name):
        return getattr(attn_module, f"{name}_proj").bias

    block.weights = Weights(w("q"), w("k"), w("v"), w("o"), m, block.rotation,
                            q_bias=b("q"), k_bias=b("k"), v_bias=b("v"), o_bias=b("o"), ctx=block.ctx)
    return KernelAttention(block, layer_idx=layer_idx)


def graft(model, layers, **kw) -> dict:
    """torch_llama.py:206-219: replace model.model.layers[i].self_attn for each i;
    returns the replaced modules, so the graft can be undone."""
    original = {}
    for i in layers:
        layer = model.model.layers[i]
        original[i] = layer.self_attn
        layer.self_attn = build_from_layer(layer.self_attn, model.config, layer_idx=i, **kw)
    return original


def ungraft(model, original: dict) -> None:
    for i, module in original.items():
        model.model.layers[i].self_attn = module


def compare_against_original(model, layer_idx: int, hidden_states, **kw):
    """torch_llama.py:226-253: one layer both ways on the same input, and the difference."""
    layer = model.model.layers[layer_idx]
    with torch.no_grad():
        ref = layer.self_attn(hidden_states, **kw)
        ref = ref[0] if isinstance(ref, tuple) else ref
    adapter = build_from_layer(layer.self_attn, model.config, layer_idx=layer_idx)
    with torch.no_grad():
        got = adapter(hidden_states, **kw)[0]
    a = ref.detach().cpu().float().numpy()
    b = got.detach().cpu().float().numpy()
    denom = max(float(np.abs(a).max()), 1e-9)
    return {
        "max_abs": float(np.abs(a - b).max()),
        "relative": float(np.abs(a - b).max() / denom),
        "cosine": float((a.ravel() @ b.ravel()) / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-30)),
        "report": adapter.last_report,
    }
