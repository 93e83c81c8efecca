"""ctypes binding of ``libyufhip.so`` (the C ABI in ``include/yuf_engine.h``).

The library is built in-tree (``python -m yufmusicgen_amd.build``).  There is
no fallback: if the library is missing or fails to load, every call raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("YUF_LIB", _PKG / "libyufhip.so"))

c_float_p = ctypes.POINTER(ctypes.c_float)
c_int32_p = ctypes.POINTER(ctypes.c_int32)
c_void_p = ctypes.c_void_p


class YufError(RuntimeError):
    """A C-ABI call returned a non-zero yuf_status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[yuf status {status}] {message}")
        self.status = status


class ModelConfigC(ctypes.Structure):
    _fields_ = [
        ("vocab_size", ctypes.c_int32), ("d_model", ctypes.c_int32), ("n_layers", ctypes.c_int32),
        ("n_heads", ctypes.c_int32), ("head_size", ctypes.c_int32), ("rosa_size", ctypes.c_int32),
        ("low_rank", ctypes.c_int32), ("tie_embeddings", ctypes.c_int32), ("dropout", ctypes.c_float),
        ("midi_offset", ctypes.c_int32), ("midi_vocab_size", ctypes.c_int32),
    ]


class RngC(ctypes.Structure):
    _fields_ = [("mt", ctypes.c_uint32 * 624), ("index", ctypes.c_uint32)]


# name -> (restype, argtypes)
SIGNATURES = {
    "yuf_last_error": (ctypes.c_char_p, []),
    "yuf_version": (ctypes.c_char_p, []),
    "yuf_wkv7_scan_f32": (ctypes.c_int, [ctypes.c_int] * 4 + [c_void_p] * 10),
    "yuf_rosa_scan_f32": (ctypes.c_int, [ctypes.c_int] * 3 + [c_void_p] * 9),
    "yuf_rosa_scan_f32_noalloc": (ctypes.c_int, [ctypes.c_int] * 3 + [c_void_p] * 9),
    "yuf_linear_f32": (ctypes.c_int, [ctypes.c_int] * 3 + [c_void_p] * 3 + [ctypes.c_int] + [c_void_p] * 3),
    "yuf_ln_linear_f32": (ctypes.c_int, [ctypes.c_int] * 3 + [c_void_p] * 9),
    "yuf_x3_planes_elems": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int]),
    "yuf_engine_time_wkv_step": (ctypes.c_int, [c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_float),
                                                ctypes.POINTER(ctypes.c_int)]),
    "yuf_x3_split_planes": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, c_void_p, c_void_p, c_void_p]),
    "yuf_linear_f32_planes": (ctypes.c_int, [ctypes.c_int] * 3 + [c_void_p] * 4 + [ctypes.c_int] + [c_void_p] * 3),
    "yuf_linear_bf16w": (ctypes.c_int, [ctypes.c_int] * 3 + [c_void_p] * 3 + [ctypes.c_int] + [c_void_p] * 3),
    "yuf_ln_linear_bf16w": (ctypes.c_int, [ctypes.c_int] * 3 + [c_void_p] * 9),
    "yuf_ckpt_load": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(c_void_p)]),
    "yuf_ckpt_free": (None, [c_void_p]),
    "yuf_ckpt_config": (ctypes.c_int, [c_void_p, ctypes.POINTER(ModelConfigC)]),
    "yuf_ckpt_tensor": (ctypes.c_int, [c_void_p, ctypes.c_char_p, ctypes.POINTER(c_float_p),
                                       ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int32),
                                       ctypes.POINTER(ctypes.c_int64)]),
    "yuf_ckpt_header_json": (ctypes.c_int, [c_void_p, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_size_t),
                                            ctypes.POINTER(ctypes.c_uint32)]),
    "yuf_engine_take_error": (ctypes.c_int, [c_void_p]),
    "yuf_engine_create": (ctypes.c_int, [c_void_p, ctypes.c_int, ctypes.c_int, ctypes.POINTER(c_void_p)]),
    "yuf_engine_create_ex": (ctypes.c_int, [c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(c_void_p)]),
    "yuf_engine_destroy": (None, [c_void_p]),
    "yuf_engine_config": (ctypes.c_int, [c_void_p, ctypes.POINTER(ModelConfigC)]),
    "yuf_engine_stream": (c_void_p, [c_void_p]),
    "yuf_prefill": (ctypes.c_int, [c_void_p, ctypes.c_int, c_void_p, ctypes.c_int, c_void_p, c_void_p, ctypes.c_int]),
    "yuf_prefill_device": (ctypes.c_int, [c_void_p, ctypes.c_int, c_void_p, ctypes.c_int, c_void_p, c_void_p,
                                          ctypes.c_int]),
    "yuf_step": (ctypes.c_int, [c_void_p, ctypes.c_int, c_void_p, c_void_p, c_void_p]),
    "yuf_step_device": (ctypes.c_int, [c_void_p, ctypes.c_int, c_void_p, c_void_p, c_void_p]),
    "yuf_state_reset": (ctypes.c_int, [c_void_p, ctypes.c_int]),
    "yuf_state_size": (ctypes.c_size_t, [c_void_p]),
    "yuf_state_save": (ctypes.c_int, [c_void_p, ctypes.c_int, c_void_p]),
    "yuf_state_load": (ctypes.c_int, [c_void_p, ctypes.c_int, c_void_p]),
    "yuf_rng_seed": (None, [ctypes.POINTER(RngC), ctypes.c_uint64]),
    "yuf_rng_next_u32": (ctypes.c_uint32, [ctypes.POINTER(RngC)]),
    "yuf_rng_next_uniform": (ctypes.c_double, [ctypes.POINTER(RngC)]),
    "yuf_sample": (ctypes.c_int32, [c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_int,
                                    ctypes.POINTER(RngC)]),
    "yuf_argmax": (ctypes.c_int32, [c_void_p, ctypes.c_int]),
    "yuf_generation_mask": (ctypes.c_int, [c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_int, c_void_p, ctypes.c_int, c_void_p]),
    "yuf_sample_device_masked": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, c_void_p, ctypes.c_float, ctypes.c_float,
                                                ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                c_void_p, c_void_p, ctypes.c_int, c_void_p, c_void_p, ctypes.c_uint64,
                                                ctypes.c_uint64, c_void_p, c_void_p]),
    "yuf_rng_exp_draws": (ctypes.c_int, [ctypes.POINTER(RngC), ctypes.c_int, ctypes.c_int, c_void_p,
                                         ctypes.POINTER(ctypes.c_int32)]),
    "yuf_sample_device": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, c_void_p, ctypes.c_float, ctypes.c_int,
                                         ctypes.c_uint64, ctypes.c_uint64, c_void_p, c_void_p]),
}

_LIB = None


def lib() -> ctypes.CDLL:
    """Load the library once; raise if it is absent (no silent fallback)."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m yufmusicgen_amd.build`")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name, None)
            if fn is None:  # reported by missing_symbols(); calling it raises AttributeError
                continue
            fn.restype = restype
            fn.argtypes = argtypes
        _LIB = handle
    return _LIB


def check(status: int) -> None:
    if status != 0:
        raise YufError(status, lib().yuf_last_error().decode("utf-8", "replace"))


def missing_symbols() -> list:
    """Declared entry points the loaded library does not export."""
    handle = lib()
    return [name for name in SIGNATURES if getattr(handle, name, None) is None]
