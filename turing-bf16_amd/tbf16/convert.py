"""Convert a bf16 model in place (tbf16/convert.py of the reference).

    tbf16.convert(model)               # inference
    tbf16.convert(pipe)                # diffusers pipeline: every nn.Module component
    tbf16.convert(model, train=True)   # training / fine-tuning (also after PEFT/LoRA wrapping)

Inference: every bf16 nn.Linear becomes a tbf16.Linear holding its weight as fp16 plus
one exact power-of-two scale per output row (same memory as bf16, same values).
Training: every nn.Linear becomes a tbf16.TrainLinear (an nn.Linear subclass, same
parameters) whose forward and backward run on fp16 MFMA for bf16 inputs.
Both route F.scaled_dot_product_attention to tbf16's scaled attention for bf16 inputs.
With conv=True (inference) every bf16 Conv1d/2d/3d becomes a scaled fp16 convolution
(tbf16.conv).
"""
import os
import warnings

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import autograd
from .attention import sdpa
from .conv import convert_conv, convertible
from .ops import prepare_weight, scaled_linear

# Train mode: linear layers with in or out features below this run in fp32 (tbf16/convert.py:26-27).
MIN_DIM = int(os.environ.get("TBF16_MIN_DIM", 128))

# Attention with fewer query rows (decoding) runs natively (tbf16/convert.py:29-30).
MIN_QUERY_ROWS = 16


class Linear(nn.Module):
    """Inference linear with fp16 weight buffers `weight16` / `weight_scale`
    (tbf16/convert.py:33-52; same buffer names, so state_dicts match)."""

    def __init__(self, lin: nn.Linear):
        super().__init__()
        self.in_features, self.out_features = lin.in_features, lin.out_features
        w16, ws = prepare_weight(lin.weight.data)
        self.register_buffer("weight16", w16)
        self.register_buffer("weight_scale", ws)
        self.bias = lin.bias

    @property
    def weight(self):  # bf16 view for code that reads .weight; materialized on demand
        return (self.weight16.float() * self.weight_scale[:, None]).bfloat16()

    def forward(self, x):
        if x.dtype != torch.bfloat16 or torch.is_grad_enabled() and x.requires_grad:
            return F.linear(x, self.weight.to(x.dtype), None if self.bias is None else self.bias.to(x.dtype))
        return scaled_linear(x, self.weight16, self.weight_scale, self.bias)

    def extra_repr(self):
        return f"in_features={self.in_features}, out_features={self.out_features}, bias={self.bias is not None}"


class TrainLinear(nn.Linear):
    """nn.Linear whose bf16 forward and backward run on fp16 MFMA. Swapped in by
    changing __class__, so parameters, hooks and PEFT wrappers are untouched
    (tbf16/convert.py:55-73)."""

    def forward(self, x):
        w, b = self.weight, self.bias
        if x.is_cuda and torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16:
            x, w = x.to(torch.bfloat16), w.to(torch.bfloat16)
            b = None if b is None else b.to(torch.bfloat16)
        if x.dtype == w.dtype == torch.bfloat16 and x.is_cuda and min(w.shape) < MIN_DIM:
            return autograd.FP32LinearFn.apply(x, w, b)
        if x.dtype == w.dtype == torch.bfloat16 and x.is_cuda and x.shape[-1] % 8 == 0:
            if torch.is_grad_enabled() and (x.requires_grad or w.requires_grad):
                return autograd.linear(x, w, b)
            return scaled_linear(x, *prepare_weight(w), b)
        return F.linear(x, w, b)


_native_sdpa = F.scaled_dot_product_attention


def _sdpa(query, key, value, *args, **kwargs):  # torch's parameter names: callers pass them as keywords
    """Router of tbf16/convert.py:79-88. bf16 4-D inputs with D <= 256 (multiple of 8)
    and at least MIN_QUERY_ROWS query rows go to tbf16 (dropout included, as the
    reference routes it); everything else runs natively."""
    q, k, v = query, key, value
    if q.is_cuda and torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16:
        q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    if (q.dtype == k.dtype == v.dtype == torch.bfloat16 and q.is_cuda and q.dim() == 4 and q.shape[-1] <= 256
            and q.shape[-1] % 8 == 0 and q.shape[-2] >= MIN_QUERY_ROWS):
        if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
            return autograd.sdpa(q, k, v, *args, **kwargs)
        return sdpa(q, k, v, *args, **kwargs)
    return _native_sdpa(q, k, v, *args, **kwargs)


def install_sdpa():
    F.scaled_dot_product_attention = _sdpa
    torch.nn.functional.scaled_dot_product_attention = _sdpa


def uninstall_sdpa():
    F.scaled_dot_product_attention = _native_sdpa


def is_supported_gpu(device=None) -> bool:
    """True on the GPU these kernels are built for: AMD Instinct MI355X (gfx950).
    (The reference answers for Volta/Turing, tbf16/convert.py:100-105; the kernels
    here are gfx950 code objects, so other GPUs cannot run them.)"""
    if not torch.cuda.is_available():
        return False
    props = torch.cuda.get_device_properties(device if device is not None else torch.cuda.current_device())
    return getattr(props, "gcnArchName", "").split(":")[0] == "gfx950"


def convert(model, train: bool = False, sdpa: bool = True, force: bool = False, conv: bool = True):
    """Convert in place and return the model (an nn.Module or a diffusers pipeline). A no-op
    (with a warning) on GPUs other than gfx950, unless force=True (tbf16/convert.py:108-147)."""
    if not force and not is_supported_gpu():
        warnings.warn("tbf16.convert: this GPU is not an MI355X (gfx950); leaving the model unchanged. "
                      "Pass force=True to convert anyway.")
        return model
    if not isinstance(model, nn.Module) and isinstance(getattr(model, "components", None), dict):
        for c in model.components.values():
            if isinstance(c, nn.Module):
                convert(c, train=train, sdpa=False, force=force, conv=conv)
        if sdpa:
            install_sdpa()
        return model
    if train:
        for mod in model.modules():
            if type(mod) is nn.Linear:
                mod.__class__ = TrainLinear
        if sdpa:
            install_sdpa()
        return model
    # A weight shared with another module (e.g. lm_head tied to the embedding) would be
    # stored twice, so those layers stay native.
    owners = {}
    for mod in model.modules():
        for p in mod.parameters(recurse=False):
            owners[id(p)] = owners.get(id(p), 0) + 1
    for name, mod in list(model.named_modules()):
        for cname, child in list(mod.named_children()):
            if (type(child) is nn.Linear and child.weight.dtype == torch.bfloat16 and child.weight.is_cuda
                    and owners[id(child.weight)] == 1):
                setattr(mod, cname, Linear(child))
                child.weight = None  # free the bf16 copy now, not when convert() returns
            elif conv and convertible(child) and owners[id(child.weight)] == 1:
                convert_conv(child)
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    if sdpa:
        install_sdpa()
    return model
