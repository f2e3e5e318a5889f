"""fp64 references evaluated with torch on whatever device the inputs are on
(the GPU for full-size configs: the CPU cannot do 1e12 fp64 FLOPs in seconds).
They are plain softmax-attention / matmul formulas in float64, the accuracy
reference the reference's own tests use (tests/test_attention.py:7-13,
tests/test_autograd.py:9-42)."""
import math

import torch


def attn_fwd64(q, k, v, causal, scale=None, bias=None, rows=None):
    """Per-(b, h) loop to bound memory; GQA by index."""
    B, H, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    idx = torch.arange(Sq, device=q.device) if rows is None else torch.as_tensor(rows, device=q.device)
    out = torch.empty(B, H, len(idx), D, dtype=torch.float64, device=q.device)
    kj = torch.arange(Sk, device=q.device)
    for b in range(B):
        for h in range(H):
            hk = h // (H // Hkv)
            s = (q[b, h, idx].double() @ k[b, hk].double().t()) * sc
            if bias is not None:
                s = s + bias[b, h, idx].double()
            if causal:
                s = s.masked_fill(kj[None, :] > idx[:, None], float("-inf"))
            out[b, h] = torch.softmax(s, -1) @ v[b, hk].double()
    return out


def attn_bwd64(q, k, v, do, causal, scale=None):
    """(o, dq, dk, dv) in fp64 from the closed-form attention gradient."""
    B, H, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    o = torch.empty(B, H, Sq, D, dtype=torch.float64, device=q.device)
    dq = torch.empty_like(o)
    dk = torch.zeros(B, Hkv, Sk, D, dtype=torch.float64, device=q.device)
    dv = torch.zeros_like(dk)
    qi = torch.arange(Sq, device=q.device)
    kj = torch.arange(Sk, device=q.device)
    for b in range(B):
        for h in range(H):
            hk = h // (H // Hkv)
            Q, K, V, dO = q[b, h].double(), k[b, hk].double(), v[b, hk].double(), do[b, h].double()
            s = (Q @ K.t()) * sc
            if causal:
                s = s.masked_fill(kj[None, :] > qi[:, None], float("-inf"))
            p = torch.softmax(s, -1)
            O = p @ V
            dp = dO @ V.t()
            delta = (dO * O).sum(-1, keepdim=True)
            ds = p * (dp - delta)
            o[b, h] = O
            dq[b, h] = (ds @ K) * sc
            dk[b, hk] += (ds.t() @ Q) * sc
            dv[b, hk] += p.t() @ dO
    return o, dq, dk, dv


def rel(y, ref):
    y, ref = y.double(), ref.double()
    return float((y - ref).norm() / ref.norm())
