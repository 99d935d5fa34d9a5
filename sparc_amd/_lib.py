"""ctypes binding of libsparc_hip.so (the C ABI declared in include/sparc_hip.h).

The library is loaded from this package directory.  There is no fallback: if
the library is missing, or no GPU is present, every compute entry point
raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libsparc_hip.so")

SPARC_F32, SPARC_BF16 = 0, 1
TRANSITIONS = {"p1": 0, "polar": 1, "cartesian": 2, "real": 3}
FLAG_RELU_OUTPUT = 1
FLAG_RESET_FIRST = 2
FLAG_ALGO_LOOKBACK = 4
FLAG_ALGO_CHAIN = 8
FLAG_ALGO_SERIAL = 16
ALGO_FLAGS = {"auto": 0, "lookback": FLAG_ALGO_LOOKBACK, "chain": FLAG_ALGO_CHAIN,
              "serial": FLAG_ALGO_SERIAL}

# every symbol declared in include/sparc_hip.h
EXPORTED_SYMBOLS = (
    "sparc_scan_chunk_length",
    "sparc_scan_chunk_count",
    "sparc_scan_workspace_bytes",
    "sparc_scan_forward",
    "sparc_scan_backward",
    "sparc_scan_workspace_error",
    "sparc_set_wait_limit",
    "sparc_write_forward",
    "sparc_write_workspace_bytes",
    "sparc_write_backward",
    "sparc_decode_step",
    "sparc_decode_workspace_bytes",
    "sparc_decode_prepare",
    "sparc_decode_step_prepared",
    "sparc_decode_step_prepared_noalloc",
    "sparc_scan_step",
    "sparc_column_sum",
    "sparc_mixer_workspace_bytes",
    "sparc_mixer_forward",
    "sparc_mixer_backward",
    "sparc_mixer_backward_form",
    "sparc_mixer_backward_plan",
    "sparc_mixer_scan_forward",
    "sparc_mixer_scan_backward",
    "sparc_controls_forward",
    "sparc_controls_workspace_bytes",
    "sparc_controls_backward",
    "sparc_controls_fold_workspace_bytes",
    "sparc_controls_fold",
    "sparc_controls_fold_backward",
    "sparc_rms_norm_forward",
    "sparc_rms_norm_workspace_bytes",
    "sparc_rms_norm_backward",
    "sparc_last_error",
    "sparc_version",
)


class ScanDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int64),
        ("length", ctypes.c_int64),
        ("modes", ctypes.c_int64),
        ("groups", ctypes.c_int64),
        ("transition", ctypes.c_int32),
        ("io_dtype", ctypes.c_int32),
        ("gate_dtype", ctypes.c_int32),
        ("flags", ctypes.c_int32),
    ]


_lock = threading.Lock()
_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_SZ = ctypes.c_size_t


def load() -> ctypes.CDLL:
    """Loads the library (once) and declares the argument types."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built: run `python -m sparc_amd.build` "
                "(the SPARC operators have no CPU fallback)")
        lib = ctypes.CDLL(LIB_PATH)
        D = ctypes.POINTER(ScanDesc)
        lib.sparc_scan_chunk_length.argtypes = [D]
        lib.sparc_scan_chunk_length.restype = _I64
        lib.sparc_scan_chunk_count.argtypes = [D]
        lib.sparc_scan_chunk_count.restype = _I64
        lib.sparc_scan_workspace_bytes.argtypes = [D, ctypes.c_int]
        lib.sparc_scan_workspace_bytes.restype = _SZ
        lib.sparc_scan_forward.argtypes = [D] + [_P] * 13 + [_SZ, _P]
        lib.sparc_scan_forward.restype = ctypes.c_int
        lib.sparc_scan_backward.argtypes = [D] + [_P] * 25 + [_SZ, _P]
        lib.sparc_scan_backward.restype = ctypes.c_int
        lib.sparc_scan_workspace_error.argtypes = [_P, _P]
        lib.sparc_scan_workspace_error.restype = ctypes.c_int
        lib.sparc_set_wait_limit.argtypes = [ctypes.c_uint32]
        lib.sparc_set_wait_limit.restype = ctypes.c_uint32
        lib.sparc_write_forward.argtypes = [_I64, _I64, _I32] + [_P] * 10
        lib.sparc_write_forward.restype = ctypes.c_int
        lib.sparc_write_workspace_bytes.argtypes = [_I64, _I64]
        lib.sparc_write_workspace_bytes.restype = _SZ
        lib.sparc_write_backward.argtypes = [_I64, _I64, _I32] + [_P] * 17 + [_SZ, _P]
        lib.sparc_write_backward.restype = ctypes.c_int
        lib.sparc_decode_step.argtypes = [_I64, _I64, _I32] + [_P] * 14
        lib.sparc_decode_step.restype = ctypes.c_int
        lib.sparc_decode_workspace_bytes.argtypes = [_I64, _I64]
        lib.sparc_decode_workspace_bytes.restype = _SZ
        lib.sparc_decode_prepare.argtypes = [_I64] + [_P] * 6 + [_P]
        lib.sparc_decode_prepare.restype = ctypes.c_int
        lib.sparc_decode_step_prepared.argtypes = [_I64, _I64, _I32] + [_P] * 9 + [_P, _SZ, _P]
        lib.sparc_decode_step_prepared.restype = ctypes.c_int
        lib.sparc_decode_step_prepared_noalloc.argtypes = [_I64, _I64, _I32] + [_P] * 9 + [_P]
        lib.sparc_decode_step_prepared_noalloc.restype = ctypes.c_int
        lib.sparc_scan_step.argtypes = [D] + [_P] * 10 + [_P]
        lib.sparc_scan_step.restype = ctypes.c_int
        lib.sparc_column_sum.argtypes = [_I64, _I64, _P, _P, ctypes.c_int, _P]
        lib.sparc_column_sum.restype = ctypes.c_int
        lib.sparc_mixer_workspace_bytes.argtypes = [_I64, _I64, _I64, ctypes.c_int]
        lib.sparc_mixer_workspace_bytes.restype = _SZ
        lib.sparc_mixer_forward.argtypes = [_I64, _I64, _I64, _I32] + [_P] * 16 + [_SZ, _P]
        lib.sparc_mixer_forward.restype = ctypes.c_int
        lib.sparc_mixer_backward.argtypes = [_I64, _I64, _I64, _I32] + [_P] * 24 + [_SZ, _P]
        lib.sparc_mixer_backward.restype = ctypes.c_int
        lib.sparc_mixer_backward_form.argtypes = [_I64, _I64, _I64, _I32]
        lib.sparc_mixer_backward_form.restype = ctypes.c_int
        lib.sparc_mixer_backward_plan.argtypes = [ctypes.c_int]
        lib.sparc_mixer_backward_plan.restype = ctypes.c_int
        lib.sparc_mixer_scan_forward.argtypes = [_I64, _I64, _I64, _I32] + [_P] * 14 + [_SZ, _P]
        lib.sparc_mixer_scan_forward.restype = ctypes.c_int
        lib.sparc_mixer_scan_backward.argtypes = [_I64, _I64, _I64, _I32] + [_P] * 22 + [_SZ, _P]
        lib.sparc_mixer_scan_backward.restype = ctypes.c_int
        lib.sparc_controls_forward.argtypes = [_I64, _I64, _I32] + [_P] * 6
        lib.sparc_controls_forward.restype = ctypes.c_int
        lib.sparc_controls_workspace_bytes.argtypes = [_I64, _I64]
        lib.sparc_controls_workspace_bytes.restype = _SZ
        lib.sparc_controls_backward.argtypes = [_I64, _I64, _I32] + [_P] * 11 + [_SZ, _P]
        lib.sparc_controls_backward.restype = ctypes.c_int
        lib.sparc_controls_fold_workspace_bytes.argtypes = [_I64, _I64]
        lib.sparc_controls_fold_workspace_bytes.restype = _SZ
        lib.sparc_controls_fold.argtypes = [_I64, _I64, _I32] + [_P] * 6 + [_SZ, _P]
        lib.sparc_controls_fold.restype = ctypes.c_int
        lib.sparc_controls_fold_backward.argtypes = [_I64, _I64, _I32] + [_P] * 8 + [_P]
        lib.sparc_controls_fold_backward.restype = ctypes.c_int
        lib.sparc_rms_norm_forward.argtypes = [_I64, _I64, _I32, _P, _P, ctypes.c_float, _P, _P, _P]
        lib.sparc_rms_norm_forward.restype = ctypes.c_int
        lib.sparc_rms_norm_workspace_bytes.argtypes = [_I64, _I64]
        lib.sparc_rms_norm_workspace_bytes.restype = _SZ
        lib.sparc_rms_norm_backward.argtypes = [_I64, _I64, _I32] + [_P] * 7 + [_SZ, _P]
        lib.sparc_rms_norm_backward.restype = ctypes.c_int
        lib.sparc_last_error.argtypes = []
        lib.sparc_last_error.restype = ctypes.c_char_p
        lib.sparc_version.argtypes = []
        lib.sparc_version.restype = ctypes.c_char_p
        _lib = lib
        return lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().sparc_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (sparc_status {status}): {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    """The device address the C ABI reads: only for contiguous tensors (the
    kernels index them as dense row-major arrays)."""
    if t is None:
        return None
    if not t.is_contiguous():
        raise ValueError("SPARC HIP kernels take contiguous tensors")
    return t.data_ptr()


def expect(t: torch.Tensor | None, shape: tuple, dtype: torch.dtype, name: str) -> None:
    """Raise ValueError unless ``t`` has this shape and dtype (the sizes the
    kernels assume: a tensor smaller than its descriptor would be read or
    written past its end)."""
    if t is None:
        raise ValueError(f"{name} is required")
    if tuple(t.shape) != tuple(shape) or t.dtype != dtype:
        raise ValueError(f"{name} must be {list(shape)} {dtype}, got {list(t.shape)} {t.dtype}")


def check_params(width: int, **named: torch.Tensor) -> None:
    """Module parameters against the input width 2M they are used with:
    ``*direction`` tensors hold width + 1 entries (bias last), every other
    (per-mode) parameter width // 2.  ValueError otherwise: the kernels read
    that many values from each."""
    for name, t in named.items():
        n = width + 1 if name.endswith("direction") else width // 2
        if t.ndim != 1 or t.numel() != n:
            raise ValueError(f"{name} must have {n} entries for inputs of width {width}, got {list(t.shape)}")


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def io_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return SPARC_F32
    if dtype == torch.bfloat16:
        return SPARC_BF16
    raise TypeError(f"SPARC HIP kernels take float32 or bfloat16 tensors, got {dtype}")


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "SPARC HIP operators need GPU tensors (this build has no CPU path); "
                f"got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError("SPARC operator inputs are on different devices")
    return dev
