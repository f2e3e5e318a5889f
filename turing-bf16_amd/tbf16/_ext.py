"""Loads the HIP library (libtbf16_hip.so) through its C ABI.

Replaces the reference's JIT pybind11 build (tbf16/_ext.py:44-107). There is no
fallback backend: if the library is missing or cannot load, every kernel call
raises, naming the build command. The library binds to the HIP runtime torch
has already loaded (same soname), so torch's device pointers and streams are
passed straight through.
"""
from __future__ import annotations

import ctypes
import pathlib

import torch

_LIB_PATH = pathlib.Path(__file__).resolve().parent / "_lib" / "libtbf16_hip.so"
ABI_VERSION = 3

DT_BF16, DT_F16 = 0, 1

_lib = None
_failed: Exception | None = None

P = ctypes.c_void_p
I = ctypes.c_int
I64 = ctypes.c_int64
F = ctypes.c_float
SZ = ctypes.c_size_t
U64 = ctypes.c_uint64
PI64 = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); mirrors include/tbf16_hip.h
_SIGS = {
    "tbf16_abi_version": (I, []),
    "tbf16_last_error": (ctypes.c_char_p, []),
    "tbf16_row_exps": (I, [P, I64, I64, I64, I, I, P, P, P]),
    "tbf16_quantize_rows": (I, [P, I64, I64, I64, I, I, P, I64, P, P]),
    "tbf16_quantize_rows_t": (I, [P, I64, I64, I64, I, P, I64, P, P, P]),
    "tbf16_quantize_cols_ws_bytes": (SZ, [I64, I64]),
    "tbf16_quantize_cols_t": (I, [P, I64, I64, I64, I, P, P, I64, P, P, I64, P]),
    "tbf16_linear_ws_bytes": (SZ, [I64, I64, I64, I]),
    "tbf16_linear": (I, [P, I64, I64, I64, P, I64, I64, P, P, P, I64, I, I, I, P, P]),
    "tbf16_linear_noalloc": (I, [P, I64, I64, I64, P, I64, I64, P, P, P, I64, I, I, I, P]),
    "tbf16_linear_exps": (I, [P, I64, I64, I64, P, P, I64, I64, P, P, P, I64, I, P]),
    "tbf16_gemm_f16": (I, [P, I64, I64, I64, P, P, I64, I64, P, P, P, I64, I, P]),
    "tbf16_gemv": (I, [P, P, I64, I64, I64, P, P, P, P]),
    "tbf16_head_amax": (I, [P, I, I64, I64, I64, I64, I64, I64, I64, P, P]),
    "tbf16_head_scale_cast": (I, [P, I, I64, I64, I64, I64, I64, I64, I64, P, I64, I64, P, I, P]),
    "tbf16_conv_input_ws_bytes": (SZ, [I64, I64]),
    "tbf16_conv_input": (I, [P, I64, I64, I, P, P, P, I64, P]),
    "tbf16_conv_epilogue": (I, [P, I64, I64, I64, I, P, P, P, P, P]),
    "tbf16_attn_fwd_ws_bytes": (SZ, [I64, I64, I64, I64, I64, I64]),
    "tbf16_attn_fwd": (I, [P, P, P, I64, I64, I64, I64, I64, I64, PI64, PI64, PI64, P, PI64, F, I, I, F, U64, P, P, P, P,
                           P, I64, P]),
    "tbf16_attn_bwd_ws_bytes": (SZ, [I64, I64, I64, I64, I64, I64]),
    "tbf16_attn_bwd": (I, [P, P, P, P, P, P, P, I64, I64, I64, I64, I64, I64, PI64, PI64, PI64, PI64, P, PI64, F,
                           I, I, F, U64, P, P, P, P, P, P, P, I64, P]),
}


def lib_path() -> pathlib.Path:
    return _LIB_PATH


def lib():
    """The loaded library; raises RuntimeError if it is not built or not loadable."""
    global _lib, _failed
    if _lib is not None:
        return _lib
    if not _LIB_PATH.exists():
        raise RuntimeError(f"tbf16: HIP library not built ({_LIB_PATH} missing). "
                           "Build it with `python turing-bf16_amd/build.py` (needs hipcc).")
    L = ctypes.CDLL(str(_LIB_PATH))
    for name, (res, args) in _SIGS.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    v = L.tbf16_abi_version()
    if v != ABI_VERSION:
        raise RuntimeError(f"tbf16: library ABI {v} != expected {ABI_VERSION}; rebuild it")
    _lib = L
    return _lib


def available() -> bool:
    """True if the HIP library loads. Unlike the reference there is no fallback:
    a False here means tbf16's ops raise."""
    global _failed
    try:
        lib()
        return True
    except Exception as e:  # noqa: BLE001
        _failed = e
        return False


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().tbf16_last_error().decode(errors="replace")
        raise RuntimeError(f"tbf16: {msg}")


_raw_stream = torch._C._cuda_getCurrentRawStream


def launch(name: str, where, *args) -> None:
    """Calls entry point `name` with `args` followed by torch's current stream on the
    device of `where` (a tensor or a torch.device). Every launching entry point takes
    its stream last. The device guard is entered only when that device is not the
    current one, which keeps a decode-sized call's host cost to a few microseconds."""
    fn = getattr(lib(), name)
    dev = where.get_device() if isinstance(where, torch.Tensor) else where.index
    if dev is None or dev < 0:
        raise ValueError("tbf16: expected tensors on a ROCm (cuda) device")
    if torch.cuda.current_device() != dev:
        with torch.cuda.device(dev):
            rc = fn(*args, _raw_stream(dev))
    else:
        rc = fn(*args, _raw_stream(dev))
    if rc != 0:
        msg = lib().tbf16_last_error().decode(errors="replace")
        raise RuntimeError(f"tbf16: {msg}")


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream() -> int:
    """torch's current HIP stream on the current device (a hipStream_t)."""
    return torch.cuda.current_stream().cuda_stream


def strides3(t) -> ctypes.Array:
    """(b, h, s) element strides of a 4-D tensor as an int64[3]."""
    s = t.stride()
    return (ctypes.c_int64 * 3)(s[0], s[1], s[2])
