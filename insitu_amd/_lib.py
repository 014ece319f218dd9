"""ctypes binding of libinsitu_hip.so (include/insitu.h).

There is no fallback: if the library is missing or fails to load, every GPU
entry point raises. The numpy model is never used to produce a product value.
"""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libinsitu_hip.so")

OK, EBADLEN, ERANGE, EHIP, EINVAL, ECAPACITY, ENOMEM, EFAULT = range(8)
SEQUENTIAL, TWO_PASS, SPLIT, SERIAL = range(4)
DEBUG_DECODE_CALLS, DEBUG_PREFILL_CALLS, DEBUG_SPIN_LIMIT, DEBUG_PATH, DEBUG_APPEND = 1, 2, 3, 4, 5
PATH_AUTO, PATH_SCAN, PATH_CHUNKED, PATH_STEP = 0, 1, 2, 3
MODES = {"online": SEQUENTIAL, "sequential": SEQUENTIAL, "two_pass": TWO_PASS,
         "split": SPLIT, "serial": SERIAL}

STATUS_NAMES = {OK: "OK", EBADLEN: "EBADLEN", ERANGE: "ERANGE", EHIP: "EHIP",
                EINVAL: "EINVAL", ECAPACITY: "ECAPACITY", ENOMEM: "ENOMEM", EFAULT: "EFAULT"}

EXPORTS = (
    "insitu_ctx_create", "insitu_ctx_destroy", "insitu_ctx_sync", "insitu_ctx_stream",
    "insitu_ctx_timing", "insitu_ctx_timing_read", "insitu_ctx_timing_read_each",
    "insitu_rotate", "insitu_encode", "insitu_qtab", "insitu_exp_lut", "insitu_finalize",
    "insitu_cache_create", "insitu_cache_destroy", "insitu_cache_reset", "insitu_cache_length",
    "insitu_cache_set_length", "insitu_cache_layout", "insitu_append", "insitu_append_seq",
    "insitu_append_wire", "insitu_attend", "insitu_attend_causal", "insitu_attend_causal_head", "insitu_attend_causal_static", "insitu_step", "insitu_project", "insitu_seam_wire",
    "insitu_project_seam",
    "insitu_output_projection", "insitu_read_rows", "insitu_load_rows", "insitu_read_image",
    "insitu_load_image", "insitu_probe_read", "insitu_probe_empty", "insitu_cache_debug",
    "insitu_cache_stats",
    "insitu_debug_scratch_layout", "insitu_last_error",
)


class InsituError(RuntimeError):
    def __init__(self, status: int, msg: str) -> None:
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


class CapacityError(InsituError, ValueError):
    """Raised where cache/base.py:67-73 raises ValueError."""


class FormatError(InsituError, ValueError):
    """Raised where config.py raises ValueError on an unsupported format."""


class Format(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "head_dim", "key_bits", "value_bits", "norm_bits", "norm_frac", "qk_frac", "qk_width",
        "centroid_frac", "acc_frac", "acc_width", "score_width", "prob_frac", "exp_lut_bits",
        "rot_rounds")] + [("rot_signs", (ctypes.c_uint64 * 2) * 8)]


class CacheDesc(ctypes.Structure):
    _fields_ = [("capacity", ctypes.c_int64), ("batch", ctypes.c_int32),
                ("n_kv_heads", ctypes.c_int32), ("n_q_heads", ctypes.c_int32),
                ("chunk_tokens", ctypes.c_int32), ("fmt", Format),
                ("key_centroids_host", ctypes.POINTER(ctypes.c_int64)),
                ("key_bounds_host", ctypes.POINTER(ctypes.c_int64)),
                ("value_centroids_host", ctypes.POINTER(ctypes.c_int64)),
                ("value_bounds_host", ctypes.POINTER(ctypes.c_int64))]


class Layout(ctypes.Structure):
    _fields_ = [("row_bytes", ctypes.c_int32), ("n_planes", ctypes.c_int32),
                ("plane_lo", ctypes.c_int32 * 16), ("plane_width", ctypes.c_int32 * 16),
                ("plane_span", ctypes.c_int64), ("head_stride", ctypes.c_int64),
                ("seq_stride", ctypes.c_int64), ("total_bytes", ctypes.c_int64),
                ("device_base", ctypes.c_uint64)]


class Stats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in (
        "n_tokens", "rescale_events", "score_overflows", "acc_overflows", "max_abs_score",
        "max_abs_acc", "range_errors", "serial_fallbacks")]


_lib = None


def load(path: str | None = None):
    """Load the library once. Raises (never falls back) when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise ImportError(f"{p} is not built; run `python -m insitu_amd.build` "
                          f"(there is no CPU fallback)")
    lib = ctypes.CDLL(p)
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    P = ctypes.POINTER
    sig = {
        "insitu_ctx_create": (i32, [i32, vp, P(vp)]),
        "insitu_ctx_destroy": (i32, [vp]),
        "insitu_ctx_sync": (i32, [vp]),
        "insitu_ctx_stream": (vp, [vp]),
        "insitu_ctx_timing": (i32, [vp, i32]),
        "insitu_ctx_timing_read": (i32, [vp, P(ctypes.c_double), P(i64)]),
        "insitu_ctx_timing_read_each": (i32, [vp, P(ctypes.c_double), i64, P(i64)]),
        "insitu_rotate": (i32, [vp, vp, vp, i64, P(Format)]),
        "insitu_encode": (i32, [vp, vp, i64, P(Format), P(i64), i32, vp, vp]),
        "insitu_qtab": (i32, [vp, vp, i32, i32, P(i64), i32, vp]),
        "insitu_exp_lut": (i32, [vp, vp, i64, vp]),
        "insitu_finalize": (i32, [vp, vp, vp, i32, i32, vp, vp, vp]),
        "insitu_cache_create": (i32, [vp, P(CacheDesc), P(vp)]),
        "insitu_cache_destroy": (i32, [vp]),
        "insitu_cache_reset": (i32, [vp]),
        "insitu_cache_length": (i32, [vp, i32, P(i64)]),
        "insitu_cache_set_length": (i32, [vp, i32, i64]),
        "insitu_cache_layout": (i32, [vp, P(Layout)]),
        "insitu_append": (i32, [vp, vp, vp, i32]),
        "insitu_append_seq": (i32, [vp, i32, vp, vp, i32]),
        "insitu_append_wire": (i32, [vp, i32, vp, vp, i32]),
        "insitu_attend": (i32, [vp, vp, vp, i32, P(Stats)]),
        "insitu_attend_causal": (i32, [vp, i32, i64, i64, vp, vp, i32, P(Stats)]),
        "insitu_attend_causal_head": (i32, [vp, i32, i32, i64, i64, vp, vp, i32, P(Stats)]),
        "insitu_attend_causal_static": (i32, [vp, i32, i64, i64, vp, vp, i32]),
        "insitu_project": (i32, [vp, vp, i32, i32, vp, i64, vp, vp]),
        "insitu_seam_wire": (i32, [vp, vp, vp, i64, i32, i32, i32, vp, i64, vp, vp, i64, i32,
                                   ctypes.c_double, i32, vp, vp, vp, P(ctypes.c_uint64)]),
        "insitu_project_seam": (i32, [vp, vp, i32, vp, i64, vp, i32, i32, i32, vp, i64, vp, vp, i64, i32,
                                      ctypes.c_double, i32, vp, vp, vp, vp, P(ctypes.c_uint64)]),
        "insitu_output_projection": (i32, [vp, vp, i64, i32, i32, vp, i32, vp, vp]),
        "insitu_step": (i32, [vp, vp, vp, vp, vp, i32, P(Stats)]),
        "insitu_read_rows": (i32, [vp, i32, i32, i64, i64, vp]),
        "insitu_load_rows": (i32, [vp, i32, i32, i64, i64, vp]),
        "insitu_read_image": (i32, [vp, i32, vp, i64]),
        "insitu_load_image": (i32, [vp, i32, vp, i64]),
        "insitu_probe_read": (i32, [vp, vp, i64, i32, i32, vp]),
        "insitu_probe_empty": (i32, [vp, i32, vp]),
        "insitu_cache_debug": (i32, [vp, i32, i64]),
        "insitu_cache_stats": (i32, [vp, P(Stats)]),
        "insitu_debug_scratch_layout": (i32, [i32, i64, i32, i32, i32, P(i64), i32]),
        "insitu_last_error": (ctypes.c_char_p, []),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    _lib = lib
    return lib


def check(status: int) -> None:
    if status == OK:
        return
    msg = load().insitu_last_error().decode(errors="replace")
    if status == ECAPACITY:
        raise CapacityError(status, msg)
    if status in (EINVAL, ERANGE):
        raise FormatError(status, msg)
    raise InsituError(status, msg)
