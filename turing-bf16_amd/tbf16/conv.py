"""bf16 convolutions on fp16 MIOpen kernels (tbf16/conv.py of the reference).

The weight gets one exact power-of-two scale per output channel and the input one
per sample (a convolution mixes positions, so rows cannot be scaled separately);
the convolution runs in fp16 with fp32 accumulation and the scales are undone in
one pass that writes bf16. The weight conversion is lossless; the input's is
lossless for every element within 2^14 of its sample's max (smaller ones become
fp16 subnormals, far below the output's bf16 rounding).

On MI355X the passes around the convolution are HIP kernels behind the C ABI
(tbf16_conv_input: per-sample max, exponent and scaled fp16 copy;
tbf16_conv_epilogue: both scales and the bias in one bf16-writing pass); the fp16
convolution is MIOpen's, through torch. 1x1 convolutions (stride 1, no padding,
one group) are per-pixel linear layers and go through scaled_linear, which scales
each pixel separately. Inference only: inputs that need gradients, or are not
bf16, run the native convolution on the dequantized weight (conv.py:34-38).
Converted modules get the class TBF16<their class>, the buffers weight16 and
weight_scale and the method dequantized_weight(), as in the reference.
"""
import functools
from typing import NamedTuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from ._ext import launch, lib, ptr
from .ops import _dev_check, _target_exp, prepare_weight, scaled_linear

_CONV = {1: F.conv1d, 2: F.conv2d, 3: F.conv3d}
_CHANNELS_LAST = {2: torch.channels_last, 3: torch.channels_last_3d}


def _sample_major(x: torch.Tensor, nd: int) -> torch.Tensor:
    """x itself when each sample is one dense run of memory (contiguous, or
    channels-last for 2-D/3-D) starting 16-byte aligned, else a copy that is."""
    dense = x.is_contiguous() or (nd in _CHANNELS_LAST and x.is_contiguous(memory_format=_CHANNELS_LAST[nd]))
    if not dense:
        x = x.contiguous()
    return x if x.data_ptr() % 16 == 0 else x.clone()


def scale_input(x: torch.Tensor, t: int):
    """bf16 (B, C, *spatial) -> (int32 (B,) exponents e, fp16 x * 2^-e in x's layout).
    e = frexp(max |x[b]|) - t, so the scaled max lies in [2^(t-1), 2^t) (conv.py:49-54).
    Empty samples take amax = 1 as the reference's where(amax > 0, amax, 1) does."""
    _dev_check(x)
    if x.dtype != torch.bfloat16:
        raise TypeError(f"tbf16.conv.scale_input: expected bf16, got {x.dtype}")
    nd = x.dim() - 2
    x = _sample_major(x, nd)
    B = x.shape[0]
    n = x[0].numel() if B else 0
    exps = torch.empty((B,), device=x.device, dtype=torch.int32)
    x16 = torch.empty_like(x, dtype=torch.float16)
    if B and n:
        wsb = lib().tbf16_conv_input_ws_bytes(B, n)
        ws = torch.empty(max(wsb, 16), device=x.device, dtype=torch.uint8)
        launch("tbf16_conv_input", x, ptr(x), B, n, int(t), ptr(exps), ptr(x16), ptr(ws), ws.numel())
    elif B:
        exps.fill_(1 - int(t))
    return exps, x16


def unscale_output(y16: torch.Tensor, exps: torch.Tensor, w_sinv: torch.Tensor, bias=None) -> torch.Tensor:
    """fp16 (B, O, *spatial) -> bf16 y16 * 2^e[b] * w_sinv[o] + bias[o] (conv.py:56-60)."""
    _dev_check(y16, exps, w_sinv)
    if y16.dtype != torch.float16 or exps.dtype != torch.int32 or exps.numel() != y16.shape[0]:
        raise TypeError("tbf16.conv.unscale_output: expected fp16 y16 and int32 exponents, one per sample")
    exps = exps.contiguous()
    nd = y16.dim() - 2
    y16 = _sample_major(y16, nd)
    cl = 0 if y16.is_contiguous() else 1
    B, O = y16.shape[:2]
    P = y16[0, 0].numel() if B and O else 0
    out = torch.empty_like(y16, dtype=torch.bfloat16)
    ws = w_sinv.float().contiguous()
    b = None if bias is None else bias.detach().float().contiguous()
    if out.numel():
        launch("tbf16_conv_epilogue", y16, ptr(y16), B, O, P, cl, ptr(exps), ptr(ws), ptr(b), ptr(out))
    return out


class ConvPlan(NamedTuple):
    """What convert_conv decided for one convolution."""
    target_exp: int   # the input's per-sample target exponent (_target_exp of the weight's fan-in)
    pointwise: bool   # 1x1, stride 1, unpadded, ungrouped: a per-pixel linear layer


def _pointwise(conv: nn.Module) -> bool:
    pad = conv.padding
    unpadded = pad == "valid" or (not isinstance(pad, str) and not any(pad))
    return unpadded and conv.groups == 1 and set(conv.kernel_size) == {1} and set(conv.stride) == {1}


def _run_scaled(conv: nn.Module, x: torch.Tensor, bias) -> torch.Tensor:
    """The scaled fp16 convolution of a batched bf16 input (tbf16/conv.py:39-60)."""
    plan = conv._tbf16_plan
    if plan.pointwise:
        O = conv.out_channels
        return scaled_linear(x.movedim(1, -1), conv.weight16.view(O, -1), conv.weight_scale, bias).movedim(-1, 1)
    padding = conv.padding
    if conv.padding_mode != "zeros":  # reflect / replicate / circular: pad first, convolve unpadded
        x = F.pad(x, conv._reversed_padding_repeated_twice, mode=conv.padding_mode)
        padding = 0
    exps, x16 = scale_input(x, plan.target_exp)
    y16 = _CONV[x.dim() - 2](x16, conv.weight16, None, conv.stride, padding, conv.dilation, conv.groups)
    return unscale_output(y16, exps, conv.weight_scale, bias)


class ScaledConvMixin:
    """First base of every converted convolution class TBF16<Conv class>
    (tbf16/conv.py:63-78). It overrides only _conv_forward, so a subclass whose own
    forward ends in super().forward (diffusers' causal 3-D convolutions) keeps
    working; the class it was made from stays a base, so isinstance checks hold."""

    def dequantized_weight(self) -> torch.Tensor:
        """The bf16 weight, rebuilt exactly from weight16 and weight_scale."""
        ws = self.weight_scale.reshape((-1,) + (1,) * (self.weight16.dim() - 1))
        return (self.weight16.float() * ws).to(torch.bfloat16)

    def _conv_forward(self, x, weight, bias):
        # `weight` is the removed parameter (None): the weight lives in weight16
        if x.dtype != torch.bfloat16 or (torch.is_grad_enabled() and x.requires_grad):
            # not bf16, or a gradient is wanted: the native convolution on the rebuilt weight
            b = None if bias is None else bias.to(x.dtype)
            return super()._conv_forward(x, self.dequantized_weight().to(x.dtype), b)
        if x.dim() == self.weight16.dim() - 1:  # unbatched input: one sample
            return _run_scaled(self, x.unsqueeze(0), bias).squeeze(0)
        return _run_scaled(self, x, bias)


@functools.lru_cache(maxsize=None)
def _scaled_class(cls: type) -> type:
    """TBF16<cls.__name__>: cls with ScaledConvMixin in front (one class per cls)."""
    return type(f"TBF16{cls.__name__}", (ScaledConvMixin, cls), {})


def convertible(m: nn.Module) -> bool:
    """A bf16 nn.Conv1d/2d/3d (or subclass) on the GPU that is not converted yet
    (tbf16/conv.py:81-83)."""
    w = getattr(m, "weight", None)
    return (isinstance(m, (nn.Conv1d, nn.Conv2d, nn.Conv3d)) and not isinstance(m, ScaledConvMixin)
            and isinstance(w, torch.Tensor) and w.dtype == torch.bfloat16 and w.is_cuda)


def convert_conv(conv: nn.Module):
    """Convert one bf16 nn.Conv{1,2,3}d (or subclass) in place and return it
    (tbf16/conv.py:86-103). The `weight` parameter becomes None; buffers weight16
    (fp16, the weight's shape) and weight_scale (fp32, one per output channel) hold
    it, and .dequantized_weight() rebuilds the bf16 tensor."""
    w = conv.weight.detach()
    O = w.shape[0]
    w16, ws = prepare_weight(w.reshape(O, -1))
    plan = ConvPlan(_target_exp(w[0].numel()), _pointwise(conv))
    conv.weight = None
    conv.register_buffer("weight16", w16.contiguous().view(w.shape))
    conv.register_buffer("weight_scale", ws)
    conv._tbf16_plan = plan
    conv.__class__ = _scaled_class(type(conv))
    return conv
