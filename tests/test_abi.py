"""The C-ABI library loads without a GPU, exports every symbol include/tbf16_hip.h
declares, and rejects bad arguments on the host before any launch."""
import ctypes
import pathlib
import re

import pytest
import torch  # noqa: F401  (binds the library to torch's HIP runtime)

from tbf16 import _ext

ROOT = pathlib.Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "tbf16_hip.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tbf16_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _ext.lib()
    syms = declared_symbols()
    assert len(syms) >= 17
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing
    # and the Python loader declares a signature for each
    assert set(syms) <= set(_ext._SIGS), set(syms) - set(_ext._SIGS)


def test_abi_version():
    assert _ext.lib().tbf16_abi_version() == _ext.ABI_VERSION == 3


def _err():
    return _ext.lib().tbf16_last_error().decode()


def test_host_validation_rejects_before_launch():
    L = _ext.lib()
    # K not a multiple of 8 (small_kernels.cu:278 message)
    assert L.tbf16_quantize_rows(16, 4, 12, 12, 0, 0, 16, 12, 16, None) == -1
    assert "multiples of 8" in _err()
    # misaligned pointer
    assert L.tbf16_quantize_rows(18, 4, 16, 16, 0, 0, 16, 16, 16, None) == -1
    # GEMM: N % 8
    assert L.tbf16_gemm_f16(16, 8, 16, 16, 16, 16, 12, 16, 16, None, 16, 16, -1, None) == -1
    assert "multiples of 8" in _err()
    # bad tile config
    assert L.tbf16_gemm_f16(16, 8, 16, 16, 16, 16, 8, 16, 16, None, 16, 8, 99, None) == -1
    # attention: heads not a multiple
    st = (ctypes.c_int64 * 3)(8, 8, 8)
    assert L.tbf16_attn_fwd(16, 16, 16, 1, 3, 2, 8, 8, 8, st, st, st, None, None, 1.0, 0, 0, 0.0, 0, 16, None, None, None,
                            16, 1 << 20, None) == -1
    assert "multiple of key/value heads" in _err()
    # attention: head dim
    assert L.tbf16_attn_fwd(16, 16, 16, 1, 2, 2, 8, 8, 264, st, st, st, None, None, 1.0, 0, 0, 0.0, 0, 16, None, None, None,
                            16, 1 << 20, None) == -1
    # workspace too small
    assert L.tbf16_attn_fwd(16, 16, 16, 1, 2, 2, 8, 8, 64, st, st, st, None, None, 1.0, 0, 0, 0.0, 0, 16, None, None, None,
                            16, 0, None) == -1
    assert "workspace" in _err()
    # dropout probability outside [0, 1)
    assert L.tbf16_attn_fwd(16, 16, 16, 1, 2, 2, 8, 8, 64, st, st, st, None, None, 1.0, 0, 0, 1.0, 0, 16, None, None, None,
                            16, 1 << 20, None) == -1
    assert "dropout_p" in _err()
    # backward head dim limit
    assert L.tbf16_attn_bwd(16, 16, 16, 16, 16, 16, 16, 1, 2, 2, 8, 8, 264, st, st, st, st, None, None, 1.0, 0, 5, 0.0, 0,
                            16, 16, 16, 16, 16, None, 16, 1 << 20, None) == -1
    # convolution passes: misaligned input, small workspace, null epilogue operand
    assert L.tbf16_conv_input(18, 2, 64, 0, 16, 16, 16, 1 << 10, None) == -1
    assert "aligned" in _err()
    assert L.tbf16_conv_input(16, 2, 64, 0, 16, 16, 16, 0, None) == -1
    assert "workspace" in _err()
    assert L.tbf16_conv_epilogue(16, 2, 4, 9, 0, None, 16, None, 16, None) == -1
    assert "null" in _err()
    # the no-allocation linear: rows beyond its static scratch are refused before any launch
    assert L.tbf16_linear_noalloc(16, (1 << 20) + 1, 8, 8, 16, 8, 8, 16, None, 16, 8, 15, 0, -1, None) == -1
    assert "scratch limit" in _err()
    # empty inputs launch nothing and succeed
    assert L.tbf16_conv_input(None, 0, 64, 0, None, None, None, 0, None) == 0
    assert L.tbf16_conv_epilogue(None, 0, 4, 9, 0, None, None, None, None, None) == 0


def test_workspace_sizes_monotone():
    L = _ext.lib()
    a = L.tbf16_attn_fwd_ws_bytes(1, 16, 16, 4096, 4096, 128)
    b = L.tbf16_attn_fwd_ws_bytes(1, 16, 16, 16384, 16384, 128)
    assert 0 < a <= b
    assert L.tbf16_quantize_cols_ws_bytes(8192, 6144) >= 6144 * 4
    assert L.tbf16_attn_bwd_ws_bytes(2, 16, 16, 4096, 4096, 128) >= 2 * 16 * 4096 * 4
    assert L.tbf16_conv_input_ws_bytes(3, 100000) >= 3 * 4 * 4 and L.tbf16_conv_input_ws_bytes(0, 5) == 0


def test_missing_library_raises(monkeypatch, tmp_path):
    """No fallback backend: a missing library is an error naming the build step."""
    monkeypatch.setattr(_ext, "_lib", None)
    monkeypatch.setattr(_ext, "_LIB_PATH", tmp_path / "nope.so")
    with pytest.raises(RuntimeError, match="not built"):
        _ext.lib()
    assert not _ext.available()
