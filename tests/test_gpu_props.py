"""Size-independent properties at the full sizes of the benchmark configs: configs[1]'s
4096^3 GEMM, configs[2]'s decode linears (M = 1, 16, 64, 255), configs[3]'s 16k
causal attention (where the fp64 checks only sample rows) and configs[4]'s training
linear and attention backward.

A power of two moved from an input into its scale leaves the fp16 operands the
kernels multiply unchanged: scaling a row of x by 2^s shifts that row's exponent
by -s and must scale its output row by exactly 2^s; scaling a row of w does the
same for an output column (its inverse scale carries the power); scaling a head of
v shifts ev by s and must scale that head's output by exactly 2^s; and q 2^r with
k 2^-r leaves every logit, so the output, bit for bit the same (a shifts by -r).
In the backward, a power of two on a row of dY moves that row's L1 exponent and
scales that row of dX; one common to all of dY moves every column exponent of
dY^T and scales dW. In the attention backward, a power of two on dO scales all
three gradients. (A power on a head of v is not such a property: the dO exponent
e is a maximum over heads of head_exp(dO) + ev (tbf16/autograd.py:173-176), so it
moves G, and dO16's fp16 subnormals round differently.)
The scaled inputs are exact in bf16 (checked) and each property leaves the fp16
operands the kernels multiply identical, so "exactly" means equal bits. A dropped
or misplaced exponent, a scale applied to the wrong row or column, or a second
rounding in the epilogue breaks these equalities.
"""
import pytest
import torch

import workloads as W
from tbf16 import _ext, attention, ops
import tbf16

pytestmark = pytest.mark.gpu


def _row_exps(x: torch.Tensor, t: int) -> torch.Tensor:
    M, K = x.shape
    e = torch.empty(M, dtype=torch.int32, device=x.device)
    _ext.call("tbf16_row_exps", x.data_ptr(), M, K, x.stride(0), t, 0, e.data_ptr(), None, _ext.stream())
    return e


def test_cfg2_row_and_column_powers_of_two(dev):
    x, w, _ = W.cfg2_square_gemm()
    x, w = x.to(dev), w.to(dev)
    M, K = x.shape
    N = w.shape[0]
    g = torch.Generator().manual_seed(11)
    s = torch.randint(-6, 7, (M,), generator=g).float().to(dev)
    q = torch.randint(-6, 7, (N,), generator=g).float().to(dev)
    x2f = x.float() * torch.exp2(s)[:, None]
    w2f = w.float() * torch.exp2(q)[:, None]
    x2, w2 = x2f.bfloat16(), w2f.bfloat16()
    assert torch.equal(x2.float(), x2f) and torch.equal(w2.float(), w2f)  # the scaled inputs are exact

    t = ops._target_exp(K)
    assert torch.equal(_row_exps(x2, t), _row_exps(x, t) - s.int())

    w16, ws = ops.prepare_weight(w)
    w16b, wsb = ops.prepare_weight(w2)
    assert torch.equal(w16b.view(torch.int16), w16.view(torch.int16))
    assert torch.equal(wsb, ws * torch.exp2(q))

    y = ops.scaled_linear(x, w16, ws)
    y_rows = ops.scaled_linear(x2, w16, ws)
    y_cols = ops.scaled_linear(x, w16b, wsb)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    assert torch.equal(y_rows.float(), y.float() * torch.exp2(s)[:, None])
    assert torch.equal(y_cols.float(), y.float() * torch.exp2(q)[None, :])


def test_cfg4_16k_head_powers_of_two(dev):
    q, k, v = (t.to(dev) for t in W.cfg4_attention(16384))
    B, H = q.shape[:2]
    g = torch.Generator().manual_seed(12)
    s = torch.randint(-3, 4, (B, H), generator=g).float().to(dev)
    sv = torch.exp2(s)[..., None, None]
    v2f = v.float() * sv
    v2 = v2f.bfloat16()
    assert torch.equal(v2.float(), v2f)

    o, _, _, e = attention.attn_forward(q, k, v, None, True, None, 13)
    o_v, _, _, e_v = attention.attn_forward(q, k, v2, None, True, None, 13)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all()
    # causal row 0 sees key 0 alone: P = 1, l = 1, so it is v's row 0, bit for bit
    assert torch.equal(o[:, :, 0].view(torch.int16), v[:, :, 0].view(torch.int16))
    assert torch.equal(e_v[2:], e[2:] + s.flatten().int())  # ev per head
    assert torch.equal(o_v.float(), o.float() * sv)

    r = 3
    q2, k2 = (q.float() * 2.0 ** r).bfloat16(), (k.float() * 2.0 ** -r).bfloat16()
    assert torch.equal(q2.float(), q.float() * 2.0 ** r) and torch.equal(k2.float(), k.float() * 2.0 ** -r)
    o_qk, _, _, e_qk = attention.attn_forward(q2, k2, v, None, True, None, 13)
    torch.cuda.synchronize()
    assert int(e_qk[0]) == int(e[0]) - r  # a
    assert torch.equal(o_qk.view(torch.int16), o.view(torch.int16))
    # the inference entry point (no exponents asked for) gives the same bits
    assert torch.equal(tbf16.sdpa(q, k, v, is_causal=True).view(torch.int16), o.view(torch.int16))


@pytest.mark.parametrize("M", W.CFG3_MS)
def test_cfg3_decode_row_powers_of_two(dev, M):
    w, xs = W.cfg3_small_m()
    w, x = w.to(dev), xs[M].to(dev)
    g = torch.Generator().manual_seed(13)
    s = torch.randint(-6, 7, (M,), generator=g).float().to(dev)
    x2f = x.float() * torch.exp2(s)[:, None]
    x2 = x2f.bfloat16()
    assert torch.equal(x2.float(), x2f)
    w16, ws = ops.prepare_weight(w)
    y = ops.scaled_linear(x, w16, ws)
    y2 = ops.scaled_linear(x2, w16, ws)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    assert torch.equal(y2.float(), y.float() * torch.exp2(s)[:, None])


def test_cfg5_linear_backward_powers_of_two(dev):
    from tbf16 import autograd, routing
    x, w, dy = (t.to(dev) for t in W.cfg5_train_linear())
    M, N = dy.shape
    g = torch.Generator().manual_seed(14)
    s = torch.randint(-6, 7, (M,), generator=g).float().to(dev)
    u = 5.0

    def grads(dyv):
        routing.activations.clear()
        xg, wg = x.clone().requires_grad_(), w.clone().requires_grad_()
        autograd.linear(xg, wg).backward(dyv)
        return xg.grad, wg.grad

    dx, dw = grads(dy)
    dx_rows, _ = grads((dy.float() * torch.exp2(s)[:, None]).bfloat16())
    _, dw_all = grads((dy.float() * 2.0 ** u).bfloat16())
    torch.cuda.synchronize()
    assert torch.isfinite(dx.float()).all() and torch.isfinite(dw.float()).all()
    # dX row m = dY row m times W: its L1 exponent shifts, the fp16 operand does not
    assert torch.equal(dx_rows.float(), dx.float() * torch.exp2(s)[:, None])
    # dW = dY^T X: a power of two common to all of dY moves every column exponent
    assert torch.equal(dw_all.float(), dw.float() * 2.0 ** u)


def test_cfg5_attention_backward_powers_of_two(dev):
    from tbf16 import autograd
    q, k, v, do = (t.to(dev) for t in W.cfg5_train_attention())
    u = 5.0

    def grads(dov):
        qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
        autograd.sdpa(qg, kg, vg, is_causal=True).backward(dov)
        return qg.grad, kg.grad, vg.grad

    dq, dk, dv = grads(do)
    dq_u, dk_u, dv_u = grads((do.float() * 2.0 ** u).bfloat16())
    torch.cuda.synchronize()
    assert all(torch.isfinite(t.float()).all() for t in (dq, dk, dv))
    # every gradient is linear in dO: its exponent e moves by u, G by -u, dO16 not
    for a, b in ((dq_u, dq), (dk_u, dk), (dv_u, dv)):
        assert torch.equal(a.float(), b.float() * 2.0 ** u)
