"""In-place conversion of a bf16 model to the scaled-fp16 kernels (tbf16/convert.py:1-147
of the reference: same entry points, layer classes, buffer names and thresholds).

    tbf16.convert(model)               # inference
    tbf16.convert(pipe)                # a diffusers-style pipeline: each nn.Module component
    tbf16.convert(model, train=True)   # training / fine-tuning (also after PEFT/LoRA wrapping)

Inference: each bf16 nn.Linear on the GPU is replaced by a tbf16.Linear whose weight
is stored as fp16 `weight16` plus one fp32 power-of-two inverse scale per output row,
`weight_scale` (the bytes of the bf16 weight, the same values); bf16 Conv1d/2d/3d
become scaled fp16 convolutions (tbf16.conv). Parameters shared between modules
(tied embeddings) stay native, so nothing is stored twice.
Training: each nn.Linear changes class to tbf16.TrainLinear, an nn.Linear subclass
with the same parameters, hooks and wrappers, whose bf16 forward and backward run
on the scaled kernels.
Both modes route F.scaled_dot_product_attention through routing.attention_route.
"""
from __future__ import annotations

import collections
import os
import warnings

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import autograd, routing
from .attention import sdpa as _scaled_sdpa
from .conv import convert_conv, convertible
from .ops import prepare_weight, scaled_linear

# Training: layers with in or out features below this run in fp32 (tbf16/convert.py:26-27).
MIN_DIM = int(os.environ.get("TBF16_MIN_DIM", 128))

# Attention with fewer query rows (decoding) runs natively (tbf16/convert.py:29-30).
MIN_QUERY_ROWS = routing.MIN_QUERY_ROWS


class Linear(nn.Module):
    """Inference stand-in for a bf16 nn.Linear (tbf16/convert.py:33-52). Buffers
    `weight16` (fp16, N x K) and `weight_scale` (fp32, N) carry the weight; `bias` is
    the original parameter."""

    def __init__(self, lin: nn.Linear):
        super().__init__()
        self.in_features = lin.in_features
        self.out_features = lin.out_features
        w16, ws = prepare_weight(lin.weight.data)
        self.register_buffer("weight16", w16)
        self.register_buffer("weight_scale", ws)
        self.bias = lin.bias

    @property
    def weight(self) -> torch.Tensor:
        """The bf16 weight, rebuilt (exactly) from weight16 and weight_scale on each read."""
        return (self.weight16.float() * self.weight_scale.unsqueeze(1)).to(torch.bfloat16)

    def forward(self, x):
        wants_grad = torch.is_grad_enabled() and x.requires_grad
        if x.dtype == torch.bfloat16 and not wants_grad:
            return scaled_linear(x, self.weight16, self.weight_scale, self.bias)
        # other dtypes, and inputs that need a gradient: the native op on the rebuilt weight
        bias = None if self.bias is None else self.bias.to(x.dtype)
        return F.linear(x, self.weight.to(x.dtype), bias)

    def extra_repr(self):
        return f"in_features={self.in_features}, out_features={self.out_features}, bias={self.bias is not None}"


def _train_linear(x, w, b):
    """TrainLinear's route (tbf16/convert.py:59-73): skinny layers (LoRA adapters)
    in fp32, bf16 layers with K % 8 == 0 on the scaled kernels (with autograd when
    a gradient is wanted), everything else native."""
    if not routing.bf16_on_gpu(x, w):
        return F.linear(x, w, b)
    if min(w.shape) < MIN_DIM:
        return autograd.FP32LinearFn.apply(x, w, b)
    if x.shape[-1] % 8:
        return F.linear(x, w, b)
    if torch.is_grad_enabled() and (x.requires_grad or w.requires_grad):
        return autograd.linear(x, w, b)
    return scaled_linear(x, *prepare_weight(w), b)


class TrainLinear(nn.Linear):
    """nn.Linear whose bf16 forward and backward run on fp16 MFMA. convert() swaps
    the class of existing layers, so parameters, hooks and PEFT wrappers stay."""

    def forward(self, x):
        w, b = self.weight, self.bias
        if x.is_cuda and routing.autocast_bf16():
            # fp32 master weights under bf16 autocast: make autocast's casts here,
            # differentiably, so the bf16 route applies
            x, w = x.to(torch.bfloat16), w.to(torch.bfloat16)
            b = None if b is None else b.to(torch.bfloat16)
        return _train_linear(x, w, b)


_native_sdpa = F.scaled_dot_product_attention


def _sdpa(*args, **kwargs):
    """F.scaled_dot_product_attention while installed (tbf16/convert.py:79-88): bf16
    calls the fused kernels take go to tbf16 (its autograd path when an input needs a
    gradient), every other call to torch's own op."""
    call = routing.bind_sdpa(args, kwargs)
    if call["query"].is_cuda and routing.autocast_bf16():
        for name in ("query", "key", "value"):
            call[name] = call[name].to(torch.bfloat16)
    route = routing.attention_route(call["query"], call["key"], call["value"], enable_gqa=call["enable_gqa"])
    q, k, v = call.pop("query"), call.pop("key"), call.pop("value")
    if route == "fused_grad":
        return autograd.sdpa(q, k, v, **call)
    if route == "fused":
        return _scaled_sdpa(q, k, v, **call)
    return _native_sdpa(q, k, v, **call)


def install_sdpa():
    """Route F.scaled_dot_product_attention through tbf16 (process-wide)."""
    F.scaled_dot_product_attention = _sdpa


def uninstall_sdpa():
    """Restore torch's own F.scaled_dot_product_attention."""
    F.scaled_dot_product_attention = _native_sdpa


def is_supported_gpu(device=None) -> bool:
    """True on the GPU these kernels are built for: AMD Instinct MI355X (gfx950).
    (The reference answers True for Volta/Turing, tbf16/convert.py:100-105; the
    kernels here are gfx950 code objects only.)"""
    if not torch.cuda.is_available():
        return False
    idx = torch.cuda.current_device() if device is None else device
    arch = getattr(torch.cuda.get_device_properties(idx), "gcnArchName", "")
    return arch.split(":")[0] == "gfx950"


def _roots(model) -> list:
    """The nn.Modules convert() rewrites: the model, or each nn.Module component of a
    pipeline object exposing a `components` dict (diffusers)."""
    if isinstance(model, nn.Module):
        return [model]
    parts = getattr(model, "components", None)
    if isinstance(parts, dict):
        return [m for m in parts.values() if isinstance(m, nn.Module)]
    raise TypeError(f"tbf16.convert: expected an nn.Module or a pipeline with .components, got {type(model)}")


def _shared_parameters(root: nn.Module) -> set:
    """ids of parameters registered directly on more than one module (tied weights).
    Modules are counted once each (root.modules() deduplicates), so a module reachable
    from two parents does not make its own weight look tied (tbf16/convert.py:132-136)."""
    owners = collections.Counter(id(p) for m in root.modules() for p in m.parameters(recurse=False))
    return {pid for pid, n in owners.items() if n > 1}


def _to_training(root: nn.Module) -> None:
    for m in root.modules():
        if type(m) is nn.Linear:
            m.__class__ = TrainLinear


def _to_inference(root: nn.Module, conv: bool) -> None:
    shared = _shared_parameters(root)
    replaced = {}  # a module reachable from two parents is converted once
    for parent in list(root.modules()):
        for name, child in list(parent.named_children()):
            if id(child) in replaced:
                setattr(parent, name, replaced[id(child)])
                continue
            w = getattr(child, "weight", None)
            if not isinstance(w, torch.Tensor) or id(w) in shared:
                continue
            if type(child) is nn.Linear and w.dtype == torch.bfloat16 and w.is_cuda:
                new = Linear(child)
                child.weight = None  # drop the bf16 copy as soon as the fp16 one exists
                replaced[id(child)] = new
                setattr(parent, name, new)
            elif conv and convertible(child):
                convert_conv(child)


def convert(model, train: bool = False, sdpa: bool = True, force: bool = False, conv: bool = True):
    """Convert `model` in place and return it (tbf16/convert.py:108-147). On GPUs other
    than gfx950 it warns and returns the model unchanged unless force=True.
    conv: also convert bf16 Conv1d/2d/3d (inference only)."""
    if not force and not is_supported_gpu():
        warnings.warn("tbf16.convert: this GPU is not an MI355X (gfx950); leaving the model unchanged. "
                      "Pass force=True to convert anyway.")
        return model
    for root in _roots(model):
        if train:
            _to_training(root)
        else:
            _to_inference(root, conv)
    if not train and torch.cuda.is_available():
        torch.cuda.empty_cache()
    if sdpa:
        install_sdpa()
    return model
