"""ctypes binding of libreels_hip.so (the C ABI declared in include/reels_hip.h).

The library is loaded from $REELS_HIP_LIBRARY when set, else from reels_amd/lib/libreels_hip.so,
the way the reference locates its native libraries (REELS_SENTENCEPIECE_LIBRARY,
src/models/wan21/tokenizer.jl:3-20; REELS_NCCL_LIBRARY, src/training/distributed.jl:131-138).
There is no fallback: a missing library raises ReelsHIPUnavailable.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT_LIB = os.path.join(HERE, "lib", "libreels_hip.so")

ABI_VERSION = 1
F32, BF16, F16 = 0, 1, 2
WS_FWD, WS_BWD, WS_FWD_NOALLOC = 0, 1, 2

# every symbol include/reels_hip.h declares
EXPORTS = (
    "reels_hip_abi_version",
    "reels_hip_last_error",
    "reels_hip_i8_pack",
    "reels_hip_i8_dequant",
    "reels_hip_i8lora_workspace_bytes",
    "reels_hip_i8lora_fwd",
    "reels_hip_i8lora_fwd_noalloc",
    "reels_hip_i8lora_fwd_f16",
    "reels_hip_i8lora_bwd",
    "reels_hip_i8lora_bwd_f16",
    "reels_hip_i8lora_bwd_bias",
    "reels_hip_i8lora_bwd_bias_f16",
    "reels_hip_gelu_tanh",
    "reels_hip_gelu_tanh_f16",
    "reels_hip_gelu_tanh_bwd",
    "reels_hip_gelu_tanh_bwd_f16",
    "reels_hip_i8lora_fwd_gelu",
    "reels_hip_i8lora_fwd_gelu_f16",
    "reels_hip_i8lora_bwd_gelu",
    "reels_hip_i8lora_bwd_gelu_f16",
    "reels_hip_i8lora_workspace_bytes_f32",
    "reels_hip_i8lora_fwd_f32",
    "reels_hip_i8lora_bwd_f32",
    "reels_hip_i8lora_bwd_bias_f32",
    "reels_hip_gelu_tanh_f32",
    "reels_hip_gelu_tanh_bwd_f32",
    "reels_hip_attention_workspace_bytes",
    "reels_hip_attention_fwd",
    "reels_hip_attention_bwd",
    "reels_hip_trace_start",
    "reels_hip_trace_only",
    "reels_hip_trace_stop",
    "reels_hip_trace_get",
)


class ReelsHIPUnavailable(RuntimeError):
    """The HIP library is not built or cannot be loaded."""


class ReelsHIPError(RuntimeError):
    """A reels_hip_* call returned a negative status."""

    def __init__(self, fn: str, code: int, message: str):
        super().__init__(f"{fn} failed ({code}): {message}")
        self.code = code


_lib = None


def library_path() -> str:
    return os.environ.get("REELS_HIP_LIBRARY", DEFAULT_LIB)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not os.path.exists(path):
        raise ReelsHIPUnavailable(
            f"libreels_hip.so not found at {path}; build it with `python -m reels_amd.build`")
    L = ctypes.CDLL(path)
    vp, i64, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t
    L.reels_hip_abi_version.restype = ctypes.c_int
    L.reels_hip_last_error.restype = ctypes.c_char_p
    L.reels_hip_i8_pack.argtypes = [vp, ctypes.c_int, i64, i64, i64, vp, vp, vp, vp]
    L.reels_hip_i8_pack.restype = ctypes.c_int
    L.reels_hip_i8_dequant.argtypes = [vp, vp, i64, i64, i64, ctypes.c_int, ctypes.c_int, vp, vp]
    L.reels_hip_i8_dequant.restype = ctypes.c_int
    L.reels_hip_i8lora_workspace_bytes.argtypes = [i64, i64, i64, i64, ctypes.c_int]
    L.reels_hip_i8lora_workspace_bytes.restype = sz
    L.reels_hip_i8lora_workspace_bytes_f32.argtypes = [i64, i64, i64, i64, ctypes.c_int]
    L.reels_hip_i8lora_workspace_bytes_f32.restype = sz
    for sfx in ("", "_f16", "_f32"):
        fwd, bwd = getattr(L, "reels_hip_i8lora_fwd" + sfx), getattr(L, "reels_hip_i8lora_bwd" + sfx)
        fwd.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, ctypes.c_float, vp, vp, vp, sz, vp]
        fwd.restype = ctypes.c_int
        bwd.argtypes = [vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, ctypes.c_float, vp, vp, vp,
                        vp, sz, vp]
        bwd.restype = ctypes.c_int
        bwb = getattr(L, "reels_hip_i8lora_bwd_bias" + sfx)
        bwb.argtypes = [vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, ctypes.c_float, vp, vp, vp,
                        vp, vp, sz, vp]
        bwb.restype = ctypes.c_int
        g, gb = getattr(L, "reels_hip_gelu_tanh" + sfx), getattr(L, "reels_hip_gelu_tanh_bwd" + sfx)
        g.argtypes = [vp, vp, i64, vp]
        g.restype = ctypes.c_int
        gb.argtypes = [vp, vp, vp, i64, vp]
        gb.restype = ctypes.c_int
    for sfx in ("", "_f16"):
        fg = getattr(L, "reels_hip_i8lora_fwd_gelu" + sfx)
        fg.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, ctypes.c_float, vp, vp, vp, vp,
                       sz, vp]
        fg.restype = ctypes.c_int
        bg = getattr(L, "reels_hip_i8lora_bwd_gelu" + sfx)
        bg.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, ctypes.c_float, vp, vp,
                       vp, vp, vp, sz, vp]
        bg.restype = ctypes.c_int
    L.reels_hip_i8lora_fwd_noalloc.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64,
                                               ctypes.c_float, vp, vp, vp]
    L.reels_hip_i8lora_fwd_noalloc.restype = ctypes.c_int
    ci = ctypes.c_int
    L.reels_hip_attention_workspace_bytes.argtypes = [i64, i64, i64]
    L.reels_hip_attention_workspace_bytes.restype = sz
    L.reels_hip_attention_fwd.argtypes = [vp, vp, vp, vp, ci, i64, i64, i64, i64, i64, ci, vp, vp, vp]
    L.reels_hip_attention_fwd.restype = ci
    L.reels_hip_attention_bwd.argtypes = [vp, vp, vp, vp, vp, vp, vp, ci, i64, i64, i64, i64, i64, ci,
                                          vp, vp, vp, vp, sz, vp]
    L.reels_hip_attention_bwd.restype = ci
    L.reels_hip_trace_start.argtypes = [ctypes.c_int]
    L.reels_hip_trace_start.restype = ctypes.c_int
    L.reels_hip_trace_stop.restype = ctypes.c_int
    L.reels_hip_trace_only.argtypes = [ctypes.c_char_p]
    L.reels_hip_trace_only.restype = ctypes.c_int
    L.reels_hip_trace_get.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_char_p),
                                      ctypes.POINTER(ctypes.c_float)]
    L.reels_hip_trace_get.restype = ctypes.c_int
    v = L.reels_hip_abi_version()
    if v != ABI_VERSION:
        raise ReelsHIPUnavailable(f"{path} has ABI version {v}, expected {ABI_VERSION}")
    _lib = L
    return L


def check(fn: str, rc: int) -> None:
    if rc != 0:
        msg = lib().reels_hip_last_error().decode("utf-8", "replace")
        raise ReelsHIPError(fn, rc, msg)


def trace_records():
    """(kernel name, ms) of every launch recorded since reels_hip_trace_start; call after the
    streams are synchronised."""
    L = lib()
    n = L.reels_hip_trace_stop()
    out = []
    name = ctypes.c_char_p()
    ms = ctypes.c_float()
    for i in range(n):
        check("reels_hip_trace_get", L.reels_hip_trace_get(i, ctypes.byref(name), ctypes.byref(ms)))
        out.append((name.value.decode(), float(ms.value)))
    return out
