"""ctypes binding of libvdnmi.so, the C-ABI library of hand-written gfx950 kernels.

torch is imported first on purpose: its bundled HIP runtime carries the same SONAME
(libamdhip64.so.7) that libvdnmi.so links against, so the library binds to the runtime
that owns torch's device memory and streams.

There is no fallback. A missing or stale library raises RuntimeError, and every nonzero
status from the library raises RuntimeError with the library's own message.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIBRARY_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libvdnmi.so")

_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_ptr = ctypes.c_void_p

# name -> argtypes; every entry point returns int status.
SIGNATURES = {
    "vdn_mxfp8_quantize": [_ptr, _i64, _i64, _i64, _ptr, _ptr, _ptr, _ptr],
    "vdn_mxfp8_act_quantize": [_ptr, _i64, _i64, _i64, _i32, _ptr, _ptr, _ptr, _ptr, _ptr],
    "vdn_mxfp8_prenorm_quantize": [_ptr, _i64, _i64, _i64, _ptr, _f32, _ptr, _i64, _ptr, _i64,
                                   _ptr, _i32, _ptr, _ptr, _ptr, _ptr, _ptr],
    "vdn_mxfp8_gemm": [_ptr, _ptr, _i64, _ptr, _ptr, _i64, _i64, _ptr, _ptr, _i64, _ptr, _i64,
                       _ptr, _ptr, _i64, _i64, _i64, _ptr, _ptr],
    "vdn_mxfp8_gemm_act_quantize": [_ptr, _ptr, _i64, _ptr, _ptr, _i64, _i64, _ptr, _i32, _ptr,
                                    _ptr, _i64, _i64, _ptr, _ptr],
    "vdn_vda_prepare": [_ptr, _i64, _i32, _i64, _i64, _i32, _i32, _i32, _i32, _ptr, _ptr],
    "vdn_vda_conv_prepare": [_ptr, _i32, _i64, _i64, _i32, _i32, _i32, _ptr, _ptr, _i32, _ptr,
                             _ptr],
    "vdn_vda_statistics": [_ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64,
                           _i32, _i32, _i32, _i32, _i32, _ptr, _ptr, _ptr],
    "vdn_vda_factors": [_ptr, _ptr, _ptr, _i64, _ptr, _ptr, _ptr],
    "vdn_vda_compose": [_ptr, _ptr, _i32, _ptr, _ptr, _i32, _ptr, _ptr, _ptr],
    "vdn_vda_scan": [_ptr, _ptr, _ptr, _i32, _i32, _i32, _ptr, _ptr],
    "vdn_vda_log_prefix": [_ptr, _i32, _i32, _ptr, _ptr],
    "vdn_vda_gather": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i32, _i32,
                       _i32, _i32, _ptr, _ptr],
    "vdn_vda_readout": [_ptr, _i64, _i64, _i64, _i32, _ptr, _ptr, _i32, _f32, _ptr, _i64, _i64,
                        _i64, _ptr, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _ptr],
    "vdn_vda_epilogue": [_ptr, _ptr, _i32, _f32, _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64,
                         _i32, _i32, _i32, _i32, _ptr],
    "vdn_qk_rmsnorm_rope": [_ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _i64, _ptr,
                            _i64, _f32, _ptr, _i64, _i64, _ptr, _i64, _i64, _i32, _i32, _i64,
                            _i32, _i32, _ptr, _ptr, _ptr],
    "vdn_window_attention": [_ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _i32,
                             _ptr, _ptr, _i32, _i32, _i32, _f32, _ptr, _i64, _i64, _ptr, _i64,
                             _i64, _ptr, _i64, _i64, _ptr],
    "vdn_window_attention_mxfp8": [_ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr,
                                   _i32, _ptr, _ptr, _i32, _f32, _ptr, _i64, _i64, _ptr, _f32,
                                   _ptr, _ptr, _i64, _i32, _ptr],
    "vdn_vda_readout_mxfp8": [_ptr, _i64, _i64, _i64, _i32, _ptr, _ptr, _i32, _f32, _ptr, _i64,
                              _i64, _i64, _ptr, _ptr, _i64, _i32, _i32, _i32, _i32, _ptr],
    "vdn_vda_readout_gated": [_ptr, _i64, _i64, _i64, _i32, _ptr, _ptr, _i32, _f32, _ptr, _i64,
                              _ptr, _ptr, _ptr, _i64, _i64, _i64, _ptr, _ptr, _i64, _i32, _i32,
                              _i32, _i32, _ptr],
    "vdn_gate_projection": [_ptr, _i64, _i64, _ptr, _i32, _i32, _i32, _ptr, _ptr, _ptr, _ptr,
                            _ptr, _ptr],
    "vdn_frame_alpha": [_ptr, _i32, _i32, _ptr, _ptr, _ptr, _i32, _i32, _ptr, _ptr],
    "vdn_adaln_tables": [_ptr, _i32, _i64, _i32, _i64, _ptr, _ptr, _i64, _ptr, _i64, _ptr],
}

_LOCK = threading.Lock()
_LIB = None


def load() -> ctypes.CDLL:
    """Loads libvdnmi.so once; raises RuntimeError when it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is None:
            if not os.path.exists(LIBRARY_PATH):
                raise RuntimeError(
                    f"{LIBRARY_PATH} is missing: build it with `python -c 'import __graft_entry__ "
                    "as g; g.build()'` (hipcc, gfx950). There is no non-HIP fallback.")
            lib = ctypes.CDLL(LIBRARY_PATH)
            lib.vdn_last_error.restype = ctypes.c_char_p
            lib.vdn_last_error.argtypes = []
            lib.vdn_abi_version.restype = ctypes.c_int
            for name, args in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = ctypes.c_int
            _LIB = lib
    return _LIB


def exported_symbols() -> list[str]:
    return ["vdn_last_error", "vdn_abi_version", *SIGNATURES]


class LaunchTimer:
    """Records a pair of timing events around every call of the named entry points while
    active (`with LaunchTimer({...}) as t:`). The events go on the caller's current stream,
    the stream every entry point launches on, so each pair brackets that launch; the stream's
    handle is kept with them."""

    def __init__(self, names):
        self.names = set(names)
        self.records = []

    def __enter__(self):
        _TIMERS.append(self)
        return self

    def __exit__(self, *exc):
        _TIMERS.remove(self)

    def durations(self):
        """[(name, args, milliseconds, stream handle)] after synchronising the device."""
        torch.cuda.synchronize()
        return [(n, a, s.elapsed_time(e), h) for n, a, s, e, h in self.records]


_TIMERS: list[LaunchTimer] = []


def call(name: str, *args) -> None:
    lib = load()
    timers = [t for t in _TIMERS if name in t.names]
    if timers:
        start = torch.cuda.Event(enable_timing=True)
        start.record()
    status = getattr(lib, name)(*args)
    if status != 0:
        raise RuntimeError(f"{name} failed ({status}): {lib.vdn_last_error().decode()}")
    if timers:
        end = torch.cuda.Event(enable_timing=True)
        end.record()
        handle = torch.cuda.current_stream().cuda_stream
        for t in timers:
            t.records.append((name, args, start, end, handle))


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device) -> int:
    """The caller's current HIP stream on `device` (launches never go to a private stream)."""
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise ValueError(f"{what} must be a CUDA (HIP) tensor")
