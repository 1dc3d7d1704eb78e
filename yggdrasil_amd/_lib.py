"""ctypes binding of libygg_hip.so (the C-ABI of include/ygg_hip.h).

torch is imported before the library is opened: torch ships its own HIP runtime (libamdhip64.so.7), and opening
this library first would bring in a second copy from /opt/rocm. With torch loaded, the library's dependency on
libamdhip64.so.7 resolves to torch's runtime, so pointers and streams are shared.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL below, see the module docstring)

LIB_PATH = Path(__file__).resolve().parent / "libygg_hip.so"

# every entry point of include/ygg_hip.h
SYMBOLS = ("ygg_load", "ygg_load_blob", "ygg_model_info", "ygg_free", "ygg_step", "ygg_run", "ygg_run_grouped",
           "ygg_run_grouped_noalloc", "ygg_softmax", "ygg_score",
           "ygg_generate", "ygg_take_errors", "ygg_float_load", "ygg_float_run", "ygg_float_take_errors",
           "ygg_float_free", "ygg_kernel_name", "ygg_spec_stats", "ygg_last_error", "ygg_version")

ERRORS = {1: "io", 2: "format", 3: "limits", 4: "nomem", 5: "arg", 6: "token", 7: "device"}
ABI_VERSION = 11


class FloatLayer(ctypes.Structure):
    """ygg_float_layer: host float64 arrays of one layer (NULL where absent)."""
    _fields_ = [(name, ctypes.c_void_p) for name in (
        "table", "transition", "readout", "unembed", "router_embed", "router_weight", "router_bias",
        "layer_input_down", "layer_input_proj")]


class FloatDesc(ctypes.Structure):
    """ygg_float_desc."""
    _fields_ = [(name, ctypes.c_int32) for name in (
        "n_layers", "d_state", "block_size", "vocab", "classes", "router_depth", "readout_rank", "layer_input_rank",
        "router_token_dim", "router_state")] + [("output_bias", ctypes.c_void_p), ("layers", FloatLayer * 8)]


class YggInfo(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int32) for name in (
        "n_layers", "d_state", "block_size", "vocab", "vocab_pad", "router_depth", "n_experts", "readout_rank",
        "layer_input_rank", "input_rank", "shift", "factored", "group", "device", "kernel",
        "pipe_max_streams", "deep", "deep_max_streams", "flow_max_streams", "router_rounds", "spec_max_streams", "grouped")] + [
        ("file_array_bytes", ctypes.c_int64), ("device_bytes", ctypes.c_int64),
        ("gather_bytes", ctypes.c_int64 * 8)]


class YggError(RuntimeError):
    """A failed C-ABI call: .code is the YGG_ERR_* status."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"{msg} (YGG_ERR_{ERRORS.get(code, code).upper()})")
        self.code = code


_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library; ImportError when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is not built: run `python -m yggdrasil_amd.build` (hipcc, gfx950)")
    L = ctypes.CDLL(str(LIB_PATH))
    vp, i32 = ctypes.c_void_p, ctypes.c_int
    L.ygg_load.argtypes = [ctypes.c_char_p, i32, ctypes.POINTER(vp)]
    L.ygg_load_blob.argtypes = [vp, ctypes.c_size_t, i32, ctypes.POINTER(vp)]
    L.ygg_model_info.argtypes = [vp, ctypes.POINTER(YggInfo)]
    L.ygg_free.argtypes = [vp]
    L.ygg_free.restype = None
    L.ygg_step.argtypes = [vp, vp, vp, vp, vp, vp, i32, vp]
    L.ygg_run.argtypes = [vp, vp, i32, i32, vp, vp, vp, vp, vp, vp]
    L.ygg_run_grouped.argtypes = [vp, vp, i32, i32, vp, vp, vp, vp, vp, vp]
    L.ygg_run_grouped_noalloc.argtypes = [vp, vp, i32, i32, vp, vp, vp, vp, vp, vp]
    L.ygg_softmax.argtypes = [vp, ctypes.c_int64, i32, vp, vp, vp]
    L.ygg_score.argtypes = [vp, vp, vp, i32, i32, vp, vp, vp]
    L.ygg_generate.argtypes = [vp, vp, i32, i32, vp, ctypes.c_float, i32, ctypes.c_uint64, vp, vp, vp]
    L.ygg_take_errors.argtypes = [vp, vp, ctypes.POINTER(ctypes.c_uint32)]
    L.ygg_kernel_name.argtypes = [vp, i32, i32, i32, ctypes.c_char_p, ctypes.c_size_t]
    L.ygg_spec_stats.argtypes = [vp, ctypes.POINTER(ctypes.c_uint64), i32]
    L.ygg_float_load.argtypes = [ctypes.POINTER(FloatDesc), i32, i32, ctypes.POINTER(vp)]
    L.ygg_float_run.argtypes = [vp, vp, i32, i32, vp, vp, vp, vp, vp]
    L.ygg_float_take_errors.argtypes = [vp, vp, ctypes.POINTER(ctypes.c_uint32)]
    L.ygg_float_free.argtypes = [vp]
    L.ygg_float_free.restype = None
    L.ygg_last_error.argtypes = []
    L.ygg_last_error.restype = ctypes.c_char_p
    L.ygg_version.argtypes = []
    if L.ygg_version() != ABI_VERSION:
        raise ImportError(f"{LIB_PATH}: ABI version {L.ygg_version()}, expected {ABI_VERSION}; rebuild")
    _lib = L
    return L


def check(rc: int) -> None:
    if rc:
        raise YggError(rc, lib().ygg_last_error().decode())
