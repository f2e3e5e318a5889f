"""GPU parity of the exported helpers the reference's tests and callers use, bit for
bit against the CPU oracle: head_scale_cast (every dtype pair, broadcast exponent
strides, results in fp16's subnormals and past its range), head_amax (bf16 and
fp16, strided layouts), the attention API helpers head_exp / head_scale /
prepare_qkv and ops.quantize_rows_shared (values and sharing); plus the caller
layer's routes that need a GPU: convert(train=True) forward and backward, a
pipeline's .components, shapes the kernels do not take (native) and head dims
that are not a multiple of 8 (zero-padded), and dropout near p = 1."""
import importlib
import math

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

import tbf16
import tbf16.autograd as ag
from oracle import tbf16_oracle as O
from tbf16 import _ext, attention, ops, routing

from _ref64 import attn_bwd64, attn_fwd64, rel

cmod = importlib.import_module("tbf16.convert")  # the package rebinds tbf16.convert to the function

pytestmark = pytest.mark.gpu

G = lambda s: torch.Generator().manual_seed(s)  # noqa: E731
DT = {torch.bfloat16: _ext.DT_BF16, torch.float16: _ext.DT_F16}


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


def _wide_input(B, H, S, D, dtype, seed):
    """Values spread over many binades (so that scaled copies reach fp16's subnormals
    and its overflow), some exact zeros and signed values."""
    g = G(seed)
    x = torch.randn(B, H, S, D, generator=g) * torch.ldexp(torch.ones(B, H, S, 1),
                                                          torch.randint(-12, 12, (B, H, S, 1), generator=g).float())
    x[..., ::7] = 0.0
    return x.to(dtype)


def _scale_cast_c_abi(x, e, out_dtype):
    """Calls tbf16_head_scale_cast through the C ABI with e's own (broadcast) strides."""
    B, H, S, D = x.shape
    y = torch.empty(B, H, S, D, dtype=out_dtype, device=x.device)
    _ext.call("tbf16_head_scale_cast", x.data_ptr(), DT[x.dtype], B, H, S, D, x.stride(0), x.stride(1), x.stride(2),
              e.data_ptr(), e.stride(0), e.stride(1), y.data_ptr(), DT[out_dtype], _ext.stream())
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("in_dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("out_dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bcast", ["full", "per_head", "per_batch", "scalar"])
def test_head_scale_cast_bit_exact(dev, in_dt, out_dt, bcast):
    B, H, S, D = 2, 3, 40, 64
    x = _wide_input(B, H, S, D, in_dt, seed=1)
    # exponents from -24 to +20: fp16 results run from subnormal (and flushed to 0)
    # to overflow (inf), bf16 results stay finite
    full = torch.tensor([[-24, 20, -10], [18, -22, 5]], dtype=torch.int32)
    e = {"full": full, "per_head": full[:1].expand(B, H), "per_batch": full[:, :1].expand(B, H),
         "scalar": full[:1, :1].expand(B, H)}[bcast]
    want = O.head_scale(x, e, out_dt)
    ed = e.to(dev) if bcast == "full" else {"per_head": full[:1].to(dev).expand(B, H),
                                           "per_batch": full[:, :1].to(dev).expand(B, H),
                                           "scalar": full[:1, :1].to(dev).expand(B, H)}[bcast]
    got = _scale_cast_c_abi(x.to(dev), ed, out_dt)
    assert np.array_equal(bits(got), bits(want)), (in_dt, out_dt, bcast)
    if out_dt == torch.float16 and bcast in ("full", "per_head", "per_batch"):  # both ends of fp16's range
        wf = want.float()
        assert torch.isinf(wf).any() and ((wf != 0) & (wf.abs() < 2.0 ** -14)).any()
    # the Python helper, on a permuted (non-contiguous) view: same bits
    xp = x.to(dev).transpose(1, 2).contiguous().transpose(1, 2)
    got2 = attention.head_scale(xp, ed, out_dt)
    assert got2.is_contiguous() and np.array_equal(bits(got2), bits(want))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_head_amax_standalone(dev, dtype):
    """tbf16_head_amax on its own (one chunk per head at small S, several at large S),
    bf16 and fp16 inputs, a permuted layout and an all-zero head."""
    for (B, H, S, D) in ((2, 3, 5, 16), (1, 4, 3000, 128)):
        x = _wide_input(B, H, S, D, dtype, seed=3 + S)
        x[0, 1] = 0
        want = O.head_amax(x)
        xd = x.to(dev)
        got = attention.head_amax(xd)
        assert torch.equal(got.cpu(), want), (dtype, S)
        perm = xd.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)  # (b, s, h) memory order
        assert perm.stride(1) == D and torch.equal(attention.head_amax(perm).cpu(), want)
        assert torch.equal(attention.head_exp(xd).cpu(), O.head_exp(x))


def test_prepare_qkv_helpers(dev):
    """attention.prepare_qkv / head_exp / expand_heads against the oracle, bit for bit,
    with GQA and heads whose logits would overflow fp16 unscaled."""
    g = G(4)
    q = (torch.randn(2, 8, 64, 64, generator=g) * torch.ldexp(torch.ones(1, 8, 1, 1),
                                                             torch.arange(8).float()[None, :, None, None])).bfloat16()
    k = (torch.randn(2, 2, 64, 64, generator=g) * 2.0 ** 11).bfloat16()
    v = (torch.randn(2, 2, 64, 64, generator=g) * 2.0 ** -6).bfloat16()
    for v_exp in (0, 13):
        q16, k16, v16, a, ev = attention.prepare_qkv(q.to(dev), k.to(dev), v.to(dev), v_exp)
        oq, ok, ov, oa, oev = O.prepare_qkv(q, k, v, v_exp)
        assert int(a) == oa and torch.equal(ev.cpu(), oev)
        for got, want in ((q16, oq), (k16, ok), (v16, ov)):
            assert got.dtype == torch.float16 and np.array_equal(bits(got), bits(want))
        assert torch.equal(attention.expand_heads(ev, 8).cpu(), O.expand_heads(oev, 8))
    # unscaled fp16 logits could overflow: the 2^a / 2^-a split is doing work here
    assert float(q.float().abs().max()) * float(k.float().abs().max()) > 65504


@pytest.mark.parametrize("l1", [False, True])
def test_quantize_rows_shared(dev, l1):
    """Values equal quantize_rows of x viewed as (-1, K) at the reference's targets,
    bit for bit; a second call on the same tensor returns the same objects; an
    in-place change of x is seen."""
    g = G(5)
    x = (torch.randn(3, 50, 264, generator=g) * torch.ldexp(torch.ones(3, 50, 1),
                                                            torch.randint(-20, 20, (3, 50, 1), generator=g).float())
         ).bfloat16().to(dev)
    t = ops.L1_TARGET if l1 else ops._target_exp(264)
    y16, s = ops.quantize_rows_shared(x, l1=l1)
    wy, ws = O.quantize_rows(x.cpu().reshape(-1, 264), t, l1)
    assert np.array_equal(bits(y16), bits(wy)) and torch.equal(s.cpu(), ws)
    y16b, sb = ops.quantize_rows_shared(x, l1=l1)
    assert y16b is y16 and sb is s
    x.mul_(2)
    y16c, sc = ops.quantize_rows_shared(x, l1=l1)
    assert y16c is not y16 and torch.equal(sc.cpu(), ws * 2)  # twice the max: half the scale


# ---- the caller layer on the GPU -----------------------------------------------------

class _Block(nn.Module):
    def __init__(self, D=256, Hd=64):
        super().__init__()
        self.Hd = Hd
        self.qkv = nn.Linear(D, 3 * D)
        self.up = nn.Linear(D, 512)
        self.down = nn.Linear(512, D, bias=False)
        self.lora = nn.Linear(D, 16, bias=False)  # skinny: the fp32 route

    def forward(self, x):
        B, S, D = x.shape
        h = D // self.Hd
        q, k, v = self.qkv(x).view(B, S, 3, h, self.Hd).permute(2, 0, 3, 1, 4)
        o = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        x = x + o.transpose(1, 2).reshape(B, S, D)
        return x + self.down(F.gelu(self.up(x))) + self.lora(x).sum(-1, keepdim=True)


def test_convert_train_forward_backward(dev):
    """convert(train=True): every nn.Linear becomes a TrainLinear (same parameters),
    F.scaled_dot_product_attention goes through tbf16's autograd path; forward and
    all parameter/input gradients within 2e-2 of an fp64 copy of the model (the bf16
    model rounds every intermediate; the kernels' own precision is tested elsewhere)."""
    torch.manual_seed(0)
    m = _Block().to(dev).bfloat16()
    ref = _Block().to(dev).double()
    ref.load_state_dict({k: v.double() for k, v in m.state_dict().items()})
    x = torch.randn(2, 96, 256, generator=G(6)).bfloat16().to(dev)
    dy = torch.randn(2, 96, 256, generator=G(7)).bfloat16().to(dev)
    params = [id(p) for p in m.parameters()]
    tbf16.convert(m, train=True)
    try:
        assert all(type(l) is cmod.TrainLinear for l in (m.qkv, m.up, m.down, m.lora))
        assert [id(p) for p in m.parameters()] == params
        assert F.scaled_dot_product_attention is cmod._sdpa
        xg = x.clone().requires_grad_()
        y = m(xg)
        y.backward(dy)
        xr = x.double().requires_grad_()
        yr = ref(xr)
        yr.backward(dy.double())
        assert rel(y, yr) < 1e-2
        assert rel(xg.grad, xr.grad) < 2e-2
        for (n, p), (_, pr) in zip(m.named_parameters(), ref.named_parameters()):
            assert p.grad is not None and torch.isfinite(p.grad).all(), n
            assert rel(p.grad, pr.grad) < 2e-2, (n, rel(p.grad, pr.grad))
    finally:
        tbf16.uninstall_sdpa()


def test_convert_pipeline_components(dev):
    """A diffusers-style pipeline: each nn.Module in .components is converted, other
    entries (a scheduler object, None) are left alone (tests/test_conv.py:102-112)."""
    class FakePipe:
        def __init__(self):
            self.components = {"vae": nn.Sequential(nn.Conv2d(8, 8, 3, padding=1)).to(dev).bfloat16(),
                               "transformer": nn.Sequential(nn.Linear(8, 8)).to(dev).bfloat16(),
                               "scheduler": object(), "text_encoder": None}

    pipe = FakePipe()
    x = torch.randn(2, 8, 8, generator=G(8)).bfloat16().to(dev)
    with torch.no_grad():
        ref = pipe.components["transformer"](x)
    out = tbf16.convert(pipe, sdpa=False)
    assert out is pipe
    assert type(pipe.components["vae"][0]).__name__ == "TBF16Conv2d"
    assert isinstance(pipe.components["transformer"][0], tbf16.Linear)
    with torch.no_grad():
        y = pipe.components["transformer"](x)
    assert rel(y, ref) < 1e-2
    pipe2 = FakePipe()
    tbf16.convert(pipe2, train=True, sdpa=False)
    assert type(pipe2.components["transformer"][0]) is cmod.TrainLinear


def test_sdpa_hook_routes_unsupported_shapes_natively(dev):
    """Calls torch takes and the kernels do not (value head dim != key head dim) run
    natively through convert()'s hook and patch(), with torch's own result."""
    q = torch.randn(1, 4, 64, 64, generator=G(9)).bfloat16().to(dev)
    k = torch.randn(1, 4, 64, 64, generator=G(10)).bfloat16().to(dev)
    v = torch.randn(1, 4, 64, 128, generator=G(11)).bfloat16().to(dev)
    want = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    assert routing.attention_route(q, k, v) == "native"
    tbf16.install_sdpa()
    try:
        got = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    finally:
        tbf16.uninstall_sdpa()
    assert torch.equal(got, want)
    with torch.no_grad(), tbf16.patch() as mode:
        got2 = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    assert torch.equal(got2, want) and mode.stats["sdpa_native"] == 1 and mode.stats["sdpa"] == 0


@pytest.mark.parametrize("D", [60, 100, 4])
def test_sdpa_head_dim_not_multiple_of_8(dev, D):
    """Head dims that are not a multiple of 8 are zero-padded for the kernels: forward
    and gradients against fp64 (3e-3), the default scale from the unpadded D."""
    q = torch.randn(1, 4, 200, D, generator=G(12)).bfloat16().to(dev)
    k = torch.randn(1, 4, 200, D, generator=G(13)).bfloat16().to(dev)
    v = torch.randn(1, 4, 200, D, generator=G(14)).bfloat16().to(dev)
    do = torch.randn(1, 4, 200, D, generator=G(15)).bfloat16().to(dev)
    o = attention.sdpa(q, k, v, is_causal=True)
    assert o.shape == q.shape and rel(o, attn_fwd64(q, k, v, True)) < 3e-3
    qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
    og = ag.sdpa(qg, kg, vg, is_causal=True)
    og.backward(do)
    ro, rdq, rdk, rdv = attn_bwd64(q, k, v, do, True)
    for n, a, r in (("o", og, ro), ("dq", qg.grad, rdq), ("dk", kg.grad, rdk), ("dv", vg.grad, rdv)):
        assert a.shape == r.shape and torch.isfinite(a).all() and rel(a, r) < 3e-3, (D, n, rel(a, r))


def test_sdpa_dropout_near_one(dev):
    """dropout_p = 0.999: kept weights scaled by 1000 stay finite (the 1 / (1 - p)
    factor is applied in fp32), forward and gradients against an fp64 reference that
    applies the oracle's keep mask."""
    p, S, D, H = 0.999, 256, 64, 2
    q = torch.randn(1, H, S, D, generator=G(16)).bfloat16().to(dev)
    k = torch.randn(1, H, S, D, generator=G(17)).bfloat16().to(dev)
    v = torch.randn(1, H, S, D, generator=G(18)).bfloat16().to(dev)
    do = torch.randn(1, H, S, D, generator=G(19)).bfloat16().to(dev)
    seed = 0x5EED_0000_1234
    z = O.dropout_z(seed, 1, H, S, S, p).to(dev)
    assert (z > 0).any()

    def ref(q, k, v):
        s_ = q @ k.transpose(-1, -2) / math.sqrt(D)
        return (torch.softmax(s_, -1) * z) @ v

    o = attention.attn_forward(q, k, v, None, False, None, v_exp=13, dropout_p=p, seed=seed)[0]
    assert torch.isfinite(o).all() and rel(o, ref(q.double(), k.double(), v.double())) < 3e-3
    qd, kd, vd = (t.double().requires_grad_() for t in (q, k, v))
    ref(qd, kd, vd).backward(do.double())
    qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
    o2, lse, o16, exps = attention.attn_forward(qg.detach(), kg.detach(), vg.detach(), None, False, None, 0, True, True,
                                                dropout_p=p, seed=seed)
    dq, dk, dv, _ = ag.attn_backward(q, k, v, o16, lse, do, exps, None, 1 / math.sqrt(D), False, dropout_p=p,
                                     seed=seed)
    for n, a, r in (("dq", dq, qd.grad), ("dk", dk, kd.grad), ("dv", dv, vd.grad)):
        assert torch.isfinite(a).all() and rel(a, r) < 3e-3, (n, rel(a, r))


def _dominant_key_case(dev, S, D=64):
    """Key 0 takes 99.2% of every query's attention (logit 12.5 against 0) and dO is
    constant, so dO16 = 2^(t_do - 1) = 32 everywhere and dv16 of key 0 is about
    S * 0.992 * 32: past 65520 at S = 4096 (the reference retries once, t_do - 8),
    8127 at S = 256 (no retry)."""
    q = torch.zeros(1, 1, S, D)
    q[..., 0] = 10.0
    k = torch.zeros(1, 1, S, D)
    k[0, 0, 0, 0] = 10.0
    v = torch.randn(1, 1, S, D, generator=G(31))
    do = torch.ones(1, 1, S, D)
    return tuple(t.bfloat16().to(dev) for t in (q, k, v, do))


@pytest.mark.parametrize("overflowing", [True, False])
def test_attn_backward_device_retry_matches_host_loop(dev, overflowing):
    """The default backward decides the overflow retry on the device (a gated second
    call); its gradients and {e, G} equal, bit for bit, those of the reference's host
    loop (check='sync'), in a case that retries once and in one that does not."""
    q, k, v, do = _dominant_key_case(dev, 4096 if overflowing else 256)
    D = q.shape[-1]
    sc = 1 / math.sqrt(D)
    o, lse, o16, exps = attention.attn_forward(q, k, v, None, False, sc, 0, True, True)
    host = ag.attn_backward(q, k, v, o16, lse, do, exps, None, sc, False, check="sync")
    devc = ag.attn_backward(q, k, v, o16, lse, do, exps, None, sc, False, check="device")
    ag.check_pending(block=True)
    t_do = 12 - math.ceil(math.log2(D))
    e = int(host[3][0])
    assert int(host[3][1]) == t_do - e - (8 if overflowing else 0)
    assert torch.equal(host[3].cpu(), devc[3].cpu())
    for n, a, b in zip(("dq", "dk", "dv"), host[:3], devc[:3]):
        assert torch.isfinite(a).all() and np.array_equal(bits(a), bits(b)), n
    # dv (the gradient that overflowed) against fp64 autograd
    qd, kd, vd = (t.double().requires_grad_() for t in (q, k, v))
    (torch.softmax(qd @ kd.transpose(-1, -2) * sc, -1) @ vd).backward(do.double())
    assert rel(devc[2], vd.grad) < 3e-3, rel(devc[2], vd.grad)


def test_attn_backward_device_retry_reports_persistent_overflow(dev):
    """A non-finite dO overflows every retry: the device-mode backward returns, and
    the deferred check raises FloatingPointError as the host loop does at once."""
    q, k, v, do = _dominant_key_case(dev, 256)
    do[0, 0, 3, 5] = float("inf")
    sc = 1 / 8
    o, lse, o16, exps = attention.attn_forward(q, k, v, None, False, sc, 0, True, True)
    with pytest.raises(FloatingPointError):
        ag.attn_backward(q, k, v, o16, lse, do, exps, None, sc, False, check="sync")
    ag.attn_backward(q, k, v, o16, lse, do, exps, None, sc, False, check="device")
    with pytest.raises(FloatingPointError):
        ag.check_pending(block=True)


def test_attn_backward_device_retry_in_a_graph(dev):
    """The device-mode backward (both the first attempt and the gated retry) captured
    in a HIP graph: three replays, with eager work between them, each equal bit for
    bit to the eager result, in the case that retries once."""
    q, k, v, do = _dominant_key_case(dev, 4096)
    sc = 1 / 8
    o, lse, o16, exps = attention.attn_forward(q, k, v, None, False, sc, 0, True, True)
    want = ag.attn_backward(q, k, v, o16, lse, do, exps, None, sc, False, check="device")
    ag.check_pending(block=True)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up off the default stream, as capture wants
        ag.attn_backward(q, k, v, o16, lse, do, exps, None, sc, False, check="device")
    torch.cuda.current_stream().wait_stream(side)
    ag.check_pending(block=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        got = ag.attn_backward(q, k, v, o16, lse, do, exps, None, sc, False, check="device")
    for _ in range(3):
        torch.randn(1 << 20, device=dev).sum()  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        for n, a, b in zip(("dq", "dk", "dv", "exps"), want, got):
            assert torch.equal(a, b), n


# ---- backward exponents and the overflow retry, against the oracle -------------------

@pytest.mark.parametrize("zero_dominates", [True, False])
def test_attn_bwd_exponents_with_zero_heads(dev, zero_dominates):
    """e and G with an all-zero dO head and an all-zero V head (GQA, H = 4, Hkv = 2):
    the zero dO head enters e through its ev_q alone (head_exp 0, attention.py:25),
    deciding e when its kv head's ev is large and dO small, and not otherwise.
    Bit-exact against the oracle; gradients finite (and within the fp64 bar when
    the zero head does not decide e; when it does, the other kv head's dO16 falls
    into fp16's subnormals, as it does in the reference)."""
    g = G(61)
    B, H, Hkv, S, D = 1, 4, 2, 200, 64
    q = (torch.randn(B, H, S, D, generator=g) * 2).bfloat16()
    k = (torch.randn(B, Hkv, S, D, generator=g) * 2).bfloat16()
    v = torch.randn(B, Hkv, S, D, generator=g) * 2.0 ** 10
    v[:, 1] = 0.0  # kv head 1: ev = frexp(0) = 0
    v = v.bfloat16()
    do = torch.randn(B, H, S, D, generator=g) * (2.0 ** -20 if zero_dominates else 2.0 ** -8)
    do[:, 0 if zero_dominates else 2] = 0.0  # on kv head 0 (ev ~ 11) or 1 (ev 0)
    do = do.bfloat16()
    a_o, ev_o = O.attn_exponents(q, k, v, 0)
    e_o, t_do, G_o = O.attn_bwd_exponents(do, O.expand_heads(ev_o, H), D)
    zero_term = int(O.expand_heads(ev_o, H)[0, 0 if zero_dominates else 2])
    assert (e_o == zero_term) == zero_dominates
    qv, kv, vv, dov = (t.to(dev) for t in (q, k, v, do))
    o, lse, o16, exps = attention.attn_forward(qv, kv, vv, None, True, None, 0, True, True)
    assert int(exps[0]) == a_o and torch.equal(exps[2:].cpu().reshape(ev_o.shape), ev_o.int())
    for mode in ("sync", "device"):
        dq, dk, dv, ex = ag.attn_backward(qv, kv, vv, o16, lse, dov, exps, None, D ** -0.5, True, check=mode)
        ag.check_pending(block=True)
        assert (int(ex[0]), int(ex[1])) == (e_o, G_o), mode
        assert all(torch.isfinite(t).all() for t in (dq, dk, dv))
    if not zero_dominates:
        _, rdq, rdk, rdv = attn_bwd64(qv, kv, vv, dov, True)
        for n, a, r in (("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
            assert rel(a, r) < 3e-3, (n, rel(a, r))


def _dominant_key_gqa(dev, S, signs, D=64):
    """One kv head, len(signs) query heads; key 0 takes ~99% of every query's
    attention and query head h's dO is the constant signs[h], so each head's dv16 of
    key 0 is S * P * 32 (P = e^12.5 / (e^12.5 + S - 1)) with that sign."""
    H = len(signs)
    q = torch.zeros(1, H, S, D)
    q[..., 0] = 10.0
    k = torch.zeros(1, 1, S, D)
    k[0, 0, 0, 0] = 10.0
    v = torch.randn(1, 1, S, D, generator=G(31))
    do = torch.ones(1, H, S, D) * torch.tensor(signs, dtype=torch.float32)[None, :, None, None]
    return tuple(t.bfloat16().to(dev) for t in (q, k, v, do))


@pytest.mark.parametrize("S,signs,retries", [(1536, (1, 1), 0), (2304, (1, -1), 1)])
def test_attn_backward_gqa_retry_per_query_head(dev, S, signs, retries):
    """GQA overflow decided per query head, as the reference checks each head's
    dk16 / dv16 before summing the group (tbf16/autograd.py:176-186, 141-146):
    at S = 1536 each head's dv16 (48.9k) fits fp16 while the group sum (97.7k) does
    not -- no retry; at S = 2304 each head's 73.1k overflows while +1 and -1 heads
    cancel -- one retry. G equals the oracle's emulation of the reference (which
    checks per head), in both retry forms, and dv meets the fp64 bar."""
    q, k, v, do = _dominant_key_gqa(dev, S, signs)
    D = q.shape[-1]
    sc = 1 / math.sqrt(D)
    o, lse, o16, exps = attention.attn_forward(q, k, v, None, False, sc, 0, True, True)
    _, _, _, own_dv, (_, _, e_o, G_o) = O.sdpa_bwd_reference_arith(q, k, v, do, causal=False, scale=sc)
    t_do = 12 - math.ceil(math.log2(D))
    assert G_o == t_do - e_o - 8 * retries
    host = ag.attn_backward(q, k, v, o16, lse, do, exps, None, sc, False, check="sync")
    devc = ag.attn_backward(q, k, v, o16, lse, do, exps, None, sc, False, check="device")
    ag.check_pending(block=True)
    assert (int(host[3][0]), int(host[3][1])) == (e_o, G_o)
    assert torch.equal(host[3].cpu(), devc[3].cpu())
    for n, a, b in zip(("dq", "dk", "dv"), host[:3], devc[:3]):
        assert torch.isfinite(a).all() and np.array_equal(bits(a), bits(b)), n
    qd, kd, vd = (t.double().requires_grad_() for t in (q, k, v))
    ke, ve = kd.expand(1, len(signs), S, D), vd.expand(1, len(signs), S, D)
    (torch.softmax(qd @ ke.transpose(-1, -2) * sc, -1) @ ve).backward(do.double())
    if sum(signs):
        assert rel(devc[2], vd.grad) < 3e-3, rel(devc[2], vd.grad)


def _f32_bits(x: float) -> int:
    return int(torch.tensor([x], dtype=torch.float32).view(torch.int32)[0])


@pytest.mark.parametrize("gate_value,r", [(65520.0 * 300, 2), (float("inf"), 5), (1000.0, 0)])
def test_attn_backward_gated_call_retry_count(dev, gate_value, r):
    """A gated call given an earlier attempt's maximum x runs at t_do - 8 r, r the
    first count with x 2^(-8 r) < 65520, at most 5 (r = 2 and the cap, which no
    real first attempt here reaches), equal bit for bit to a direct call at that
    t_do; with nothing to redo (r = 0) it leaves the outputs as they are and writes
    the gate's word as its own."""
    g = G(62)
    B, H, Hkv, S, D = 1, 4, 2, 160, 64
    q, k, v = ((torch.randn(B, hh, S, D, generator=g) * 3).bfloat16().to(dev) for hh in (H, Hkv, Hkv))
    do = (torch.randn(B, H, S, D, generator=g) * 2.0 ** -10).bfloat16().to(dev)
    sc = D ** -0.5
    o, lse, o16, exps = attention.attn_forward(q, k, v, None, True, sc, 0, True, True)
    t_do = 12 - math.ceil(math.log2(D))
    args = (q, k, v, o16, lse, do, exps, None, sc, True)
    words = torch.zeros(2, device=dev, dtype=torch.int32)
    dq, dk, dv, ex, _, ws = ag._attn_backward_once(*args, t_do, overflow=words[0:1])
    first = [t.clone() for t in (dq, dk, dv, ex)]
    assert not ag._overflowed(int(words[0]))
    gate = torch.tensor([_f32_bits(gate_value)], device=dev, dtype=torch.int32)
    ag._attn_backward_once(*args, t_do, overflow=words[1:2], gate=gate, outs=(dq, dk, dv, ex), ws=ws)
    want = ag._attn_backward_once(*args, t_do - 8 * r)[:4] if r else first
    torch.cuda.synchronize()
    for n, a, b in zip(("dq", "dk", "dv", "exps"), (dq, dk, dv, ex), want):
        assert torch.equal(a, b), (n, r)
    assert int(ex[1]) == t_do - 8 * r - int(ex[0])
    if r == 0:
        assert int(words[1]) == int(gate[0])


def test_sdpa_backward_raises_on_persistent_overflow(dev, monkeypatch):
    """Device mode through autograd: a non-finite dO overflows every retry, and
    FloatingPointError comes from the backward() call itself (the end-of-backward
    check), before the gradients can reach an optimizer step."""
    monkeypatch.setattr(ag, "CHECK_OVERFLOW", "device")
    q, k, v, do = _dominant_key_gqa(dev, 256, (1, 1))
    do[0, 1, 3, 5] = float("inf")
    qd, kd, vd = (t.clone().requires_grad_() for t in (q, k, v))
    ag._pending.clear()
    with pytest.raises(FloatingPointError):
        ag.sdpa(qd, kd, vd, scale=1 / 8, enable_gqa=True).backward(do)
    assert ag._pending == []
    # a clean backward afterwards raises nothing
    q2 = q.clone().requires_grad_()
    ag.sdpa(q2, k, v, scale=1 / 8, enable_gqa=True).backward(torch.ones_like(do))
    assert torch.isfinite(q2.grad).all()
