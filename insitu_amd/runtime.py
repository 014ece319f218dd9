"""Device context and the glue between torch device memory and the C ABI.

PyTorch supplies device memory and the stream; the work is done by
libinsitu_hip.so. A Context binds the library to torch's current stream on a
device, so library kernels and torch copies are ordered on one stream.
"""

from __future__ import annotations

import ctypes
import threading

import numpy as np

from . import _lib

_contexts: dict = {}
_lock = threading.Lock()


def _torch():
    import torch
    return torch


class Context:
    """insitu_ctx_create/destroy (include/insitu.h) on one device and stream."""

    def __init__(self, device: int = 0, stream=None) -> None:
        torch = _torch()
        if not torch.cuda.is_available():
            raise RuntimeError("insitu_amd needs a ROCm GPU; there is no CPU fallback")
        self.lib = _lib.load()
        self.device = device
        self.torch_device = torch.device("cuda", device)
        with torch.cuda.device(device):
            s = stream if stream is not None else torch.cuda.current_stream(device)
        self.stream = s
        h = ctypes.c_void_p()
        _lib.check(self.lib.insitu_ctx_create(device, ctypes.c_void_p(s.cuda_stream),
                                              ctypes.byref(h)))
        self.handle = h

    def sync(self) -> None:
        _lib.check(self.lib.insitu_ctx_sync(self.handle))

    def close(self) -> None:
        if self.handle:
            self.lib.insitu_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    # -- tensors --------------------------------------------------------------

    def to_device(self, a, dtype=None):
        """numpy/torch -> contiguous torch tensor on this device (int32 by default)."""
        torch = _torch()
        if isinstance(a, torch.Tensor):
            t = a.to(self.torch_device, non_blocking=False)
        else:
            t = torch.from_numpy(np.ascontiguousarray(a)).to(self.torch_device)
        if dtype is not None:
            t = t.to(dtype)
        return t.contiguous()


def default_context(device: int = 0) -> Context:
    with _lock:
        ctx = _contexts.get(device)
        if ctx is None:
            ctx = Context(device)
            _contexts[device] = ctx
        return ctx


def ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def i64p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))
