"""ctypes view of oracle/pow2.c (test infrastructure only).

Built by `make -C oracle` (also run by __graft_entry__.build()).
"""
import ctypes
import pathlib

import numpy as np

_LIB = pathlib.Path(__file__).resolve().parent / "_build" / "libtbf16_oracle.so"
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not _LIB.exists():
            raise FileNotFoundError(f"{_LIB} missing: run `make -C oracle`")
        L = ctypes.CDLL(str(_LIB))
        P = ctypes.c_void_p
        L.tbf16o_pow2_exp_n.argtypes = [P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, P]
        L.tbf16o_scaled_f16_n.argtypes = [P, ctypes.c_int64, ctypes.c_int, P]
        L.tbf16o_f32_to_bf16_n.argtypes = [P, ctypes.c_int64, P]
        L.tbf16o_f32_to_f16_n.argtypes = [P, ctypes.c_int64, P]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def pow2_exp(amax, t, fused=False):
    a = np.ascontiguousarray(amax, dtype=np.float32).ravel()
    out = np.empty(a.shape, np.int32)
    lib().tbf16o_pow2_exp_n(_p(a), a.size, int(t), int(fused), _p(out))
    return out


def scaled_f16_bits(bf16_bits, p):
    b = np.ascontiguousarray(bf16_bits, dtype=np.uint16).ravel()
    out = np.empty(b.shape, np.uint16)
    lib().tbf16o_scaled_f16_n(_p(b), b.size, int(p), _p(out))
    return out


def f32_to_bf16_bits(x):
    a = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(a.shape, np.uint16)
    lib().tbf16o_f32_to_bf16_n(_p(a), a.size, _p(out))
    return out


def f32_to_f16_bits(x):
    a = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(a.shape, np.uint16)
    lib().tbf16o_f32_to_f16_n(_p(a), a.size, _p(out))
    return out
