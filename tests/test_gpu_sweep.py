"""Seeded shape sweeps through the public API against fp64 and the oracle.

Shapes are drawn once from a fixed seed (ragged everywhere the kernels allow:
N and K multiples of 8, D a multiple of 8 up to 256, any M, Sq, Sk), so every
run checks the same list. Each case names its shape in its test id."""
import math
import random

import numpy as np
import pytest
import torch

import tbf16
from tbf16 import ops

from _ref64 import attn_fwd64, rel
from oracle import tbf16_oracle as O

pytestmark = pytest.mark.gpu

_R = random.Random(20261201)
LINEAR_SHAPES = [(_R.choice([1, 2, 3, 17, 64, 129, 255, 256, 300, 513]), 8 * _R.randint(1, 129),
                  8 * _R.randint(1, 375)) for _ in range(24)]
ATTN_SHAPES = []
for _ in range(16):
    hkv = _R.choice([1, 2, 3])
    ATTN_SHAPES.append((_R.choice([1, 2]), hkv * _R.choice([1, 2, 4]), hkv, _R.randint(1, 700), _R.randint(1, 700),
                        8 * _R.randint(1, 32), _R.random() < 0.5))


@pytest.mark.parametrize("M,N,K", LINEAR_SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in LINEAR_SHAPES])
def test_linear_sweep(dev, M, N, K):
    """scaled_linear on the dispatcher's own path for the shape (GEMV, skinny,
    tiled; L1 or max row scales): output against fp64 at the reference's bar
    (tests/test_ops.py:25), and the row exponents the path uses bit-exact."""
    g = torch.Generator().manual_seed(M * 7919 + N * 31 + K)
    x = (torch.randn(M, K, generator=g) * torch.ldexp(torch.ones(M, 1), torch.randint(-8, 9, (M, 1), generator=g))
         ).bfloat16()
    w = (torch.randn(N, K, generator=g) / math.sqrt(K)).bfloat16()
    bias = torch.randn(N, generator=g).bfloat16()
    w16, ws = tbf16.prepare_weight(w.to(dev))
    y = tbf16.scaled_linear(x.to(dev), w16, ws, bias.to(dev))
    ref = x.double() @ w.double().t() + bias.double()
    assert y.shape == (M, N) and y.dtype == torch.bfloat16 and torch.isfinite(y).all()
    e = rel(y.cpu(), ref)
    assert e < 3e-3, e
    # the weight's exponents, and the activation's where the path scales it
    assert torch.equal(ws.cpu(), O.prepare_weight(w)[1])
    if M >= 2:
        l1 = M < ops.FUSED_MIN_M
        xd = x.to(dev)
        ex = torch.empty(M, dtype=torch.int32, device=dev)
        tbf16._ext.call("tbf16_row_exps", xd.data_ptr(), M, K, K, 15, int(l1), ex.data_ptr(), None,
                        tbf16._ext.stream())
        torch.cuda.synchronize()
        assert np.array_equal(ex.cpu().numpy(), O.row_exps(x, 15, l1))


@pytest.mark.parametrize("B,H,Hkv,Sq,Sk,D,causal", ATTN_SHAPES,
                         ids=[f"{b}x{h}/{hk}x{sq}x{sk}xD{d}{'c' if c else ''}" for b, h, hk, sq, sk, d, c in ATTN_SHAPES])
def test_attention_sweep(dev, B, H, Hkv, Sq, Sk, D, causal):
    """tbf16.sdpa (GQA when H > Hkv; causal top-left as torch's is_causal) against
    fp64 on the same bf16 inputs, at the bar of the reference's tests
    (tests/test_sdpa_api.py:39 uses 1e-2; 3e-3 here)."""
    g = torch.Generator().manual_seed(B * 1009 + H * 101 + Sq * 7 + Sk * 3 + D)
    q = (torch.randn(B, H, Sq, D, generator=g) * 2).bfloat16().to(dev)
    k = (torch.randn(B, Hkv, Sk, D, generator=g) * 2).bfloat16().to(dev)
    v = torch.randn(B, Hkv, Sk, D, generator=g).bfloat16().to(dev)
    with torch.no_grad():
        o = tbf16.sdpa(q, k, v, is_causal=causal, enable_gqa=H != Hkv)
    ref = attn_fwd64(q, k, v, False) if not causal else _causal64(q, k, v)
    assert o.shape == (B, H, Sq, D) and torch.isfinite(o).all()
    e = rel(o, ref)
    assert e < 3e-3, e


def _causal64(q, k, v):
    """fp64 attention with torch's top-left causal mask (key j visible to query i iff j <= i)."""
    B, H, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    keep = torch.ones(Sq, Sk, dtype=torch.bool, device=q.device).tril()
    out = torch.empty(B, H, Sq, D, dtype=torch.float64, device=q.device)
    for b in range(B):
        for h in range(H):
            hk = h // (H // Hkv)
            s = (q[b, h].double() @ k[b, hk].double().t()) / math.sqrt(D)
            out[b, h] = torch.softmax(s.masked_fill(~keep, float("-inf")), -1) @ v[b, hk].double()
    return out


_R2 = random.Random(20261202)
BWD_SHAPES = []
for _ in range(8):
    hkv = _R2.choice([1, 2])
    BWD_SHAPES.append((_R2.choice([1, 2]), hkv * _R2.choice([1, 2, 3]), hkv, _R2.randint(16, 600), _R2.randint(16, 600),
                       8 * _R2.randint(1, 32), _R2.random() < 0.5))
TRAIN_LINEAR_SHAPES = [(_R2.randint(2, 700), 8 * _R2.randint(1, 100), 8 * _R2.randint(1, 100)) for _ in range(6)]


def _grads(fn, inputs, dout):
    ins = [t.detach().clone().requires_grad_() for t in inputs]
    out = fn(*ins)
    out.backward(dout)
    return [out] + [t.grad for t in ins]


@pytest.mark.parametrize("B,H,Hkv,Sq,Sk,D,causal", BWD_SHAPES,
                         ids=[f"{b}x{h}/{hk}x{sq}x{sk}xD{d}{'c' if c else ''}" for b, h, hk, sq, sk, d, c in BWD_SHAPES])
def test_attention_backward_sweep(dev, B, H, Hkv, Sq, Sk, D, causal):
    """tbf16.autograd.sdpa forward and backward (dq, dk, dv with the GQA group sums)
    against fp64 autograd on the same bf16 inputs."""
    import tbf16.autograd as ag
    g = torch.Generator().manual_seed(B * 997 + H * 89 + Sq * 5 + Sk * 11 + D)
    q = torch.randn(B, H, Sq, D, generator=g).bfloat16().to(dev)
    k = torch.randn(B, Hkv, Sk, D, generator=g).bfloat16().to(dev)
    v = torch.randn(B, Hkv, Sk, D, generator=g).bfloat16().to(dev)
    do = torch.randn(B, H, Sq, D, generator=g).bfloat16().to(dev)
    keep = torch.ones(Sq, Sk, dtype=torch.bool, device=dev).tril()

    def ref(q, k, v):
        k, v = k.repeat_interleave(H // Hkv, 1), v.repeat_interleave(H // Hkv, 1)
        s = q @ k.transpose(-1, -2) / math.sqrt(D)
        if causal:
            s = s.masked_fill(~keep, float("-inf"))
        return torch.softmax(s, -1) @ v

    r = _grads(ref, [q.double(), k.double(), v.double()], do.double())
    ours = _grads(lambda q, k, v: ag.sdpa(q, k, v, is_causal=causal, enable_gqa=H != Hkv), [q, k, v], do)
    for n, o, rr in zip(["o", "dq", "dk", "dv"], ours, r):
        e = rel(o, rr)
        assert o.shape == rr.shape and torch.isfinite(o).all() and e < 3e-3, (n, e)


@pytest.mark.parametrize("M,K,N", TRAIN_LINEAR_SHAPES, ids=[f"{m}x{k}x{n}" for m, k, n in TRAIN_LINEAR_SHAPES])
def test_train_linear_sweep(dev, M, K, N):
    """tbf16.autograd.linear with bias: y, dx, dw, db against fp64 autograd."""
    import tbf16.autograd as ag
    g = torch.Generator().manual_seed(M * 13 + K * 7 + N)
    x = torch.randn(M, K, generator=g).bfloat16().to(dev)
    w = (torch.randn(N, K, generator=g) / math.sqrt(K)).bfloat16().to(dev)
    b = torch.randn(N, generator=g).bfloat16().to(dev)
    dy = (torch.randn(M, N, generator=g) * 1e-3).bfloat16().to(dev)
    r = _grads(lambda x, w, b: x @ w.t() + b, [x.double(), w.double(), b.double()], dy.double())
    ours = _grads(lambda x, w, b: ag.linear(x, w, b), [x, w, b], dy)
    for n, o, rr in zip(["y", "dx", "dw", "db"], ours, r):
        e = rel(o, rr)
        assert o.shape == rr.shape and torch.isfinite(o).all() and e < 3e-3, (n, e)
