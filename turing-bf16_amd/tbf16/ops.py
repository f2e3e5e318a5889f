"""bf16 matmuls on fp16 MFMA (MI355X / gfx950), using exact power-of-two scaling.

bf16 has an 8-bit significand and fp16 has 11, so any bf16 value inside fp16's
range converts exactly. Each row is moved into that range by a power-of-two
scale (exact), the fp16 GEMM accumulates in fp32, and the scales are undone in
the epilogue, which writes bf16 from fp32 with a single rounding.

Mirrors tbf16/ops.py of the reference (same names, arguments and results). The
kernels are hand-written HIP (turing-bf16_amd/csrc) behind a C ABI; there is no
Triton or second backend, so a missing library raises instead of falling back.
"""
from __future__ import annotations

import math
import os

import torch
import torch.nn.functional as F

from . import routing
from ._ext import available, launch, lib, ptr  # noqa: F401  (available re-exported as in the reference)

# TBF16_GEMM=fused forces the max-scaled fused path for every M >= 2 (the reference's
# switch between its fused kernel and the cuBLAS path, tbf16/ops.py:20-23). Unset:
# M >= FUSED_MIN_M uses max row scales at t = 15, smaller M the L1 row scales.
_GEMM = os.environ.get("TBF16_GEMM", "")
# TBF16_GEMM_CFG=<n> pins the GEMM tile configuration (benchmarking only).
_GEMM_CFG = int(os.environ.get("TBF16_GEMM_CFG", "-1"))
FUSED_MIN_M = 256
# Fused GEMM row scaling: max -> [2^14, 2^15) (tbf16/ops.py:24-26).
_FUSED_SCALE = (15, False)
# Rows below FUSED_MIN_M: L1 norm below 2^15 (tbf16/ops.py:129-130).
L1_TARGET = 15
# Rows below this use the GEMV kernel (tbf16/ops.py:202-204).
SMALL_M = 2


def _target_exp(K: int) -> int:
    """Target exponent t for rows whose fp16 products are summed over K terms
    (tbf16/ops.py:29-32). Both operands scaled below 2^t bound every partial sum by
    K * 2^(2t); t is the largest value <= 0 with ceil(log2 K) + 2t <= 15, i.e. the
    sum stays below 2^15 < 65504: 0 up to K = 32768, -1 up to 2^17, ..."""
    lg = math.ceil(math.log2(max(K, 1)))
    return min(0, (15 - lg) // 2)


def _dev_check(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("tbf16: expected tensors on a ROCm (cuda) device")


def _ok_rows(x: torch.Tensor) -> bool:
    """Row-major with 16-byte rows: what the kernels read without a copy."""
    return (x.dim() == 2 and x.stride(1) == 1 and x.shape[1] % 8 == 0 and x.stride(0) % 8 == 0
            and x.data_ptr() % 16 == 0)


def _pad_cols(x: torch.Tensor, mult: int = 8) -> torch.Tensor:
    """Zero-pad the last dimension to a multiple of `mult` (contiguous copy). Zeros
    change neither maxima, L1 norms nor dot products."""
    K = x.shape[-1]
    pad = (-K) % mult
    x = x.contiguous()
    return F.pad(x, (0, pad)) if pad else x


def quantize_rows(x: torch.Tensor, target_exp: int = 0, l1: bool = False):
    """bf16 (R, K) -> (fp16 (R, K), fp32 (R,) inverse scales) (tbf16/ops.py:74-89).
    Row r is multiplied by the power of two that puts its max |x| (its L1 norm with
    l1=True) in [2^(t-1), 2^t); every bf16 value then converts exactly unless its
    scaled magnitude falls below fp16's smallest normal 2^-14 (it becomes an fp16
    subnormal, rounded to nearest even)."""
    assert x.dim() == 2 and x.stride(1) == 1
    _dev_check(x)
    if x.dtype != torch.bfloat16:
        raise TypeError("tbf16.quantize_rows: expected bf16")
    R, K = x.shape
    xk = x if _ok_rows(x) else _pad_cols(x)
    Kp = xk.shape[1]
    y = torch.empty((R, Kp), device=x.device, dtype=torch.float16)
    s_inv = torch.empty((R,), device=x.device, dtype=torch.float32)
    if R:
        launch("tbf16_quantize_rows", x, ptr(xk), R, Kp, xk.stride(0), int(target_exp), int(l1), ptr(y), y.stride(0),
               ptr(s_inv))
    return (y if Kp == K else y[:, :K]), s_inv


def quantize_rows_shared(x: torch.Tensor, l1: bool = False):
    """quantize_rows(x.reshape(-1, K)) remembered per activation tensor, so the layers
    that read one activation (Q/K/V, gate/up) quantise it once (tbf16/ops.py:107-137).
    Max rows use t = _target_exp(K), L1 rows t = L1_TARGET; the memo is
    routing.activations (dropped when x is freed or modified in place)."""
    K = x.shape[-1]
    t = L1_TARGET if l1 else _target_exp(K)
    return routing.activations.get(x, ("rows", t, bool(l1)),
                                   lambda: quantize_rows(x.reshape(-1, K).contiguous(), t, l1))


def prepare_weight(w: torch.Tensor):
    """nn.Linear weight (N, K) bf16 -> (fp16 (N, K), fp32 (N,) inverse scales), rows
    max-scaled at t = _target_exp(K); done once per weight (tbf16/ops.py:140-142)."""
    return quantize_rows(w.contiguous(), _target_exp(w.shape[1]))


def _bias_bf16(bias, N, device):
    if bias is None:
        return None
    b = bias.to(device=device, dtype=torch.bfloat16).contiguous()
    if b.numel() != N:
        raise ValueError(f"tbf16: bias has {b.numel()} elements, expected {N}")
    return b


def _prep_gemm_operands(x2, w16, w_sinv, bias):
    """Pads K and N to multiples of 8 where needed (copies only then)."""
    M, K = x2.shape
    N = w16.shape[0]
    if w16.shape[1] != K:
        raise ValueError(f"tbf16: x has K={K}, weight has K={w16.shape[1]}")
    if not _ok_rows(x2):
        x2 = _pad_cols(x2)
    if not _ok_rows(w16) or w16.shape[1] != x2.shape[1]:
        w16 = _pad_cols(w16)
    ws = w_sinv.float().contiguous()
    b = _bias_bf16(bias, N, x2.device)
    Np = N + (-N) % 8
    if Np != N:
        w16 = F.pad(w16, (0, 0, 0, Np - N))
        ws = F.pad(ws, (0, Np - N), value=1.0)
        if b is not None:
            b = F.pad(b, (0, Np - N))
    return x2, w16, ws, b, N, Np


# tbf16_linear's workspace bytes per (device, M, K, N, cfg): the tile choice inside
# depends on the device's CU count, so it is asked on the tensors' device, once
_WS_BYTES: dict = {}


def _linear_ws_bytes(device: torch.device, M: int, K: int, N: int) -> int:
    key = (device.index, M, K, N, _GEMM_CFG)
    wsb = _WS_BYTES.get(key)
    if wsb is None:
        if len(_WS_BYTES) > 4096:
            _WS_BYTES.clear()
        with torch.cuda.device(device):
            wsb = _WS_BYTES[key] = int(lib().tbf16_linear_ws_bytes(M, K, N, _GEMM_CFG))
    return wsb


def _linear(x2, w16, w_sinv, bias, t, l1):
    x2, w16, ws, b, N, Np = _prep_gemm_operands(x2, w16, w_sinv, bias)
    M, Kp = x2.shape
    y = torch.empty((M, Np), device=x2.device, dtype=torch.bfloat16)
    work = torch.empty((_linear_ws_bytes(x2.device, M, Kp, Np),), device=x2.device, dtype=torch.uint8)
    launch("tbf16_linear", x2, ptr(x2), M, Kp, x2.stride(0), ptr(w16), Np, w16.stride(0), ptr(ws), ptr(b), ptr(y),
           y.stride(0), int(t), int(l1), _GEMM_CFG, ptr(work))
    return y if Np == N else y[:, :N]


def scaled_linear(x: torch.Tensor, w16: torch.Tensor, w_sinv: torch.Tensor, bias=None):
    """y = x @ W^T + b for bf16 x, with W given by prepare_weight. Returns bf16
    (tbf16/ops.py:145-164). M < 2 -> GEMV; M >= FUSED_MIN_M -> one fused kernel with
    max row scales (t = 15); 2 <= M < FUSED_MIN_M -> the same kernel with the
    reference's L1 row scales (t = 15), fp32 accumulation and no fp16 intermediate."""
    _dev_check(x, w16, w_sinv)
    shape = x.shape
    K = shape[-1]
    N = w16.shape[0]
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    if M == 0:
        return torch.empty(*shape[:-1], N, device=x.device, dtype=torch.bfloat16)
    if M < SMALL_M:
        return small_m_linear(x2, w16, w_sinv, bias).reshape(*shape[:-1], N)
    t, l1 = _FUSED_SCALE if (M >= FUSED_MIN_M or _GEMM == "fused") else (L1_TARGET, True)
    return _linear(x2, w16, w_sinv, bias, t, l1).reshape(*shape[:-1], N)


def linear_q(x16, x_sinv, w16, w_sinv, bias=None):
    """GEMM + epilogue on already-quantized rows: (x16 * x_sinv) @ (w16 * w_sinv)^T + bias,
    bf16 (M, N) (tbf16/ops.py:167-178). fp32 accumulation, one bf16 rounding (the
    reference rounds to fp16 first)."""
    _dev_check(x16, w16)
    M, K = x16.shape
    x16, w16, ws, b, N, Np = _prep_gemm_operands(x16, w16, w_sinv, bias)
    sa = x_sinv.float().contiguous()
    y = torch.empty((M, Np), device=x16.device, dtype=torch.bfloat16)
    if M:
        launch("tbf16_gemm_f16", x16, ptr(x16), M, x16.shape[1], x16.stride(0), ptr(sa), ptr(w16), Np, w16.stride(0),
               ptr(ws), ptr(b), ptr(y), y.stride(0), _GEMM_CFG)
    return y if Np == N else y[:, :N]


def small_m_linear(x2: torch.Tensor, w16: torch.Tensor, w_sinv: torch.Tensor, bias=None):
    """M = 1: GEMV in fp32 with no activation scale (tbf16/ops.py:207-218 ->
    small_kernels.cu:107-132). M >= 2: the scaled GEMM with L1 row scales."""
    M, K = x2.shape
    if M != 1:
        return _linear(x2, w16, w_sinv, bias, L1_TARGET, True)
    N = w16.shape[0]
    xk = _pad_cols(x2) if not _ok_rows(x2) else x2
    wk = _pad_cols(w16) if (not _ok_rows(w16) or w16.shape[1] != xk.shape[1]) else w16
    ws = w_sinv.float().contiguous()
    b = _bias_bf16(bias, N, x2.device)
    y = torch.empty((1, N), device=x2.device, dtype=torch.bfloat16)
    launch("tbf16_gemv", x2, ptr(xk), ptr(wk), N, wk.shape[1], wk.stride(0), ptr(ws), ptr(b), ptr(y))
    return y
