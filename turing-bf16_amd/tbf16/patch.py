"""Run unmodified bf16 PyTorch code on the scaled fp16 kernels (tbf16/patch.py:1-66 of the
reference: same context manager, mode class, threshold and stats counters).

    with tbf16.patch() as mode:
        out = model(**inputs)
    mode.stats  # {"linear": ..., "linear_native": ..., "sdpa": ..., "sdpa_native": ...}

A TorchFunctionMode that sees every F.linear and F.scaled_dot_product_attention
call while active. Inference only: with grad mode on, both run natively.
  * F.linear with bf16 GPU input and weight and at least two rows goes to
    scaled_linear; the weight's fp16 copy is made once per weight version and
    dropped when the weight is freed. Single-row calls stay native (counted as
    "linear_native").
  * F.scaled_dot_product_attention goes to tbf16.sdpa when routing.attention_route
    accepts the call (bf16, >= min_rows query rows, shapes the kernels take);
    everything else runs natively ("sdpa_native").
Every other torch function passes through untouched.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch.overrides import TorchFunctionMode

from . import routing
from .attention import sdpa
from .ops import prepare_weight, scaled_linear

# Fewer query rows than this (decoding) run attention natively (tbf16/patch.py:18-20).
MIN_ROWS = routing.MIN_QUERY_ROWS


def _bind_linear(args, kwargs):
    """(input, weight, bias) of one F.linear call, positional or by keyword."""
    names = ("input", "weight", "bias")
    call = dict(zip(names, args))
    call.update(kwargs)
    return call["input"], call["weight"], call.get("bias")


class TuringBF16Mode(TorchFunctionMode):
    """The mode patch() returns. `stats` counts routed and native calls."""

    def __init__(self, min_rows=MIN_ROWS):
        super().__init__()
        self.min_rows = min_rows
        self.stats = {"linear": 0, "linear_native": 0, "sdpa": 0, "sdpa_native": 0}
        self._weights = routing.TensorMemo()
        self._handlers = {F.linear: self._linear, F.scaled_dot_product_attention: self._attention}

    def weight16(self, w: torch.Tensor):
        """(w16, inverse scales) of weight w, made once per version of w."""
        return self._weights.get(w, "w16", lambda: prepare_weight(w.detach()))

    def _linear(self, func, args, kwargs):
        x, w, b = _bind_linear(args, kwargs)
        if routing.bf16_on_gpu(x, w) and not torch.is_grad_enabled():
            if x.dim() >= 1 and x.numel() >= 2 * max(x.shape[-1], 1):
                self.stats["linear"] += 1
                return scaled_linear(x, *self.weight16(w), b)
            self.stats["linear_native"] += 1
        return func(*args, **kwargs)

    def _attention(self, func, args, kwargs):
        call = routing.bind_sdpa(args, kwargs)
        q, k, v = call.pop("query"), call.pop("key"), call.pop("value")
        if not torch.is_grad_enabled() and routing.attention_route(
                q, k, v, enable_gqa=call["enable_gqa"], min_rows=self.min_rows, allow_grad=False) == "fused":
            self.stats["sdpa"] += 1
            return sdpa(q, k, v, **call)
        self.stats["sdpa_native"] += 1
        return func(q, k, v, **call)

    def __torch_function__(self, func, types, args=(), kwargs=None):
        handler = self._handlers.get(func)
        if handler is None:
            return func(*args, **(kwargs or {}))
        return handler(func, args, kwargs or {})


def patch(min_rows=MIN_ROWS):
    """Context manager: F.linear and F.scaled_dot_product_attention on bf16 GPU tensors
    run on the scaled fp16 kernels inside it (inference; grad mode runs natively)."""
    return TuringBF16Mode(min_rows)
