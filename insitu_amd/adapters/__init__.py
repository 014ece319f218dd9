"""Adapters that put the GPU attention block where a model's attention module was
(adapters/ of the reference)."""
