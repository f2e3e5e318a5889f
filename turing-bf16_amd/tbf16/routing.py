"""Routing decisions and per-tensor memos shared by every entry into tbf16.

Three callers intercept torch code: convert()'s layers and its SDPA hook, the
TuringBF16Mode of patch(), and the training layer TrainLinear. They all ask the
same two questions here, so a shape the kernels cannot take is sent to native
torch in every one of them instead of raising in some:

  * attention_route(q, k, v, ...): does this F.scaled_dot_product_attention call
    go to the fused kernels, and with or without autograd?
  * bf16_on_gpu(...): are these tensors bf16 on a ROCm device?

The routing thresholds are the reference's: attention with fewer than 16 query
rows (decoding) and head dims above 256 stay native (tbf16/convert.py:29-30,
83-84; tbf16/patch.py:18-20,52). Beyond them, this build also sends native
what its kernels do not compute: a value head dim different from the key's,
key/value tensors of different shapes, and batch sizes that disagree.

TensorMemo keeps results derived from a tensor (its fp16 copy and scales) for as
long as the tensor lives and is not modified in place: sibling layers fed by one
activation (Q/K/V, gate/up) quantise it once, and patch() converts each weight
once per version.
"""
from __future__ import annotations

import collections
import weakref

import torch

# attention with fewer query rows than this runs natively (tbf16/convert.py:29-30)
MIN_QUERY_ROWS = 16
# largest head dim of the fused attention kernels (tbf16/convert.py:83)
MAX_HEAD_DIM = 256


def bf16_on_gpu(*ts) -> bool:
    """Every tensor is a bf16 tensor on a ROCm (torch 'cuda') device."""
    return all(isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.bfloat16 for t in ts)


def autocast_bf16() -> bool:
    """bf16 autocast is active on the GPU: callers cast to bf16 themselves (what autocast
    would do) before deciding."""
    return torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16


def kernel_takes_qkv(q, k, v, enable_gqa: bool = False) -> str | None:
    """None if the fused attention kernels compute softmax(q k^T) v for these shapes,
    else the reason they do not. Head dims that are not a multiple of 8 are taken
    (the caller zero-pads them)."""
    if not (q.dim() == k.dim() == v.dim() == 4):
        return "expected 4-D (B, H, S, D) tensors"
    B, H, _, D = q.shape
    Bk, Hkv, _, Dk = k.shape
    if tuple(v.shape) != tuple(k.shape):
        return f"value shape {tuple(v.shape)} differs from key shape {tuple(k.shape)}"
    if Bk != B or Dk != D:
        return f"query {tuple(q.shape)} and key {tuple(k.shape)} disagree in batch or head dim"
    if Hkv != H and not (enable_gqa and Hkv > 0 and H % Hkv == 0):
        return "key/value heads differ from query heads (pass enable_gqa=True with H % Hkv == 0)"
    if D > MAX_HEAD_DIM or D == 0:
        return f"head dim {D} outside 1..{MAX_HEAD_DIM}"
    return None


def attention_route(q, k, v, enable_gqa: bool = False, min_rows: int = MIN_QUERY_ROWS,
                    allow_grad: bool = True) -> str:
    """'native', 'fused' (inference) or 'fused_grad' (autograd) for one
    scaled_dot_product_attention call on tensors that are already in the dtype the
    call will use."""
    if not bf16_on_gpu(q, k, v) or q.dim() != 4 or q.shape[-2] < min_rows:
        return "native"
    if kernel_takes_qkv(q, k, v, enable_gqa) is not None:
        return "native"
    needs_grad = torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad)
    if needs_grad:
        return "fused_grad" if allow_grad else "native"
    return "fused"


# F.scaled_dot_product_attention's parameters, in order, with their defaults
_SDPA_PARAMS = ("query", "key", "value", "attn_mask", "dropout_p", "is_causal", "scale", "enable_gqa")
_SDPA_DEFAULTS = {"attn_mask": None, "dropout_p": 0.0, "is_causal": False, "scale": None, "enable_gqa": False}


def bind_sdpa(args: tuple, kwargs: dict) -> dict:
    """The arguments of one scaled_dot_product_attention call by name (callers pass
    q, k, v positionally or as query=/key=/value=, as diffusers does)."""
    if len(args) > len(_SDPA_PARAMS):
        raise TypeError(f"scaled_dot_product_attention takes at most {len(_SDPA_PARAMS)} arguments")
    call = dict(_SDPA_DEFAULTS)
    call.update(zip(_SDPA_PARAMS, args))
    for name, val in kwargs.items():
        if name not in _SDPA_PARAMS:
            raise TypeError(f"scaled_dot_product_attention got an unexpected keyword argument '{name}'")
        if _SDPA_PARAMS.index(name) < len(args):
            raise TypeError(f"scaled_dot_product_attention got multiple values for argument '{name}'")
        call[name] = val
    for name in ("query", "key", "value"):
        if name not in call:
            raise TypeError(f"scaled_dot_product_attention missing required argument '{name}'")
    return call


class TensorMemo:
    """Values derived from tensors, each kept while its tensor is alive and at the
    version it had when the value was made.

    Entries are keyed by (id(tensor), key). A finaliser on the tensor drops its
    entries when it is freed, so a later tensor that reuses the address never sees
    them; an in-place change bumps the tensor's version and the stale value is
    rebuilt. With `capacity`, the least recently used entries beyond it are evicted.
    """

    def __init__(self, capacity: int | None = None):
        self.capacity = capacity
        self._entries: collections.OrderedDict = collections.OrderedDict()
        self._watched: dict[int, weakref.finalize] = {}

    def _forget(self, tid: int) -> None:
        self._watched.pop(tid, None)
        for key in [k for k in self._entries if k[0] == tid]:
            del self._entries[key]

    def get(self, t: torch.Tensor, key, build):
        slot = (id(t), key)
        hit = self._entries.get(slot)
        if hit is not None and hit[0] == t._version:
            self._entries.move_to_end(slot)
            return hit[1]
        value = build()
        self._entries[slot] = (t._version, value)
        self._entries.move_to_end(slot)
        if id(t) not in self._watched:
            self._watched[id(t)] = weakref.finalize(t, self._forget, id(t))
        if self.capacity is not None:
            while len(self._entries) > self.capacity:
                (tid, _), _ = self._entries.popitem(last=False)
                if not any(k[0] == tid for k in self._entries):
                    fin = self._watched.pop(tid, None)
                    if fin is not None:
                        fin.detach()
        return value

    def clear(self) -> None:
        for fin in self._watched.values():
            fin.detach()
        self._watched.clear()
        self._entries.clear()

    def __len__(self) -> int:
        return len(self._entries)


# Quantised activations: one fp16 copy of x for all the linear layers it feeds.
activations = TensorMemo(capacity=8)
