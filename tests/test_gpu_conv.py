"""Scaled convolutions on the GPU: tbf16.conv against the oracle and fp64.

Restates the reference's tests/test_conv.py (every case, its 3e-3 bar against the
fp64 convolution of the same bf16 input, the convert() and subclass checks) and
adds bit-level checks of the two HIP passes around MIOpen's fp16 convolution:
the per-sample exponents and scaled input (tbf16_conv_input) and the epilogue
(tbf16_conv_epilogue), each against the CPU oracle on the same inputs. Inputs
come from seeded CPU generators."""
import copy

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

import tbf16
from tbf16 import conv as tconv
from tbf16.conv import convert_conv

from oracle import tbf16_oracle as O

pytestmark = pytest.mark.gpu

G = lambda s: torch.Generator().manual_seed(s)  # noqa: E731
CONV = {1: F.conv1d, 2: F.conv2d, 3: F.conv3d}


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16)


def _same_bits(a, b):
    """Equal bit patterns, every NaN counted equal to every NaN."""
    a, b = a.detach().cpu(), b.detach().cpu()
    na, nb = torch.isnan(a.float()), torch.isnan(b.float())
    return torch.equal(na, nb) and torch.equal(_bits(a)[~na], _bits(b)[~nb])


# ---- the two HIP passes, bit level ---------------------------------------------------

INPUT_CASES = [
    ("nchw", (2, 64, 40, 56), False),
    ("odd n", (3, 3, 7, 9), False),          # n = 189: vectors straddle samples
    ("channels_last", (2, 24, 11, 13), True),
    ("conv1d", (5, 48, 100), False),
    ("conv3d channels_last", (1, 32, 5, 24, 40), True),
    ("many chunks", (2, 16, 64, 80), False),  # n = 81920 > one block's chunk
]


@pytest.mark.parametrize("name,shape,cl", INPUT_CASES, ids=[c[0] for c in INPUT_CASES])
@pytest.mark.parametrize("t", [0, -2])
def test_conv_input_matches_oracle(dev, name, shape, cl, t):
    g = G(11)
    B = shape[0]
    scales = torch.tensor([1e-8, 1.0, 3e4, 1e6, 0.25][:B]).view((B,) + (1,) * (len(shape) - 1))
    x = (torch.randn(shape, generator=g) * scales).bfloat16()
    xd = x.to(dev)
    if cl:
        xd = xd.to(memory_format=torch.channels_last if x.dim() == 4 else torch.channels_last_3d)
    e, x16 = tconv.scale_input(xd, t)
    torch.cuda.synchronize()
    e_ref = O.conv_sample_exps(x, t)
    assert e.cpu().numpy().tolist() == e_ref.tolist(), name
    assert x16.stride() == xd.stride()
    assert _same_bits(x16.contiguous(), O.conv_scale_input(x, e_ref)), name


def test_conv_input_edge_samples(dev):
    """All-zero, NaN, inf, bf16-subnormal and huge samples, one per batch entry;
    the subnormal sample's scale is 2^(>=128) = inf in fp32, as in the reference."""
    x = torch.randn(6, 3, 5, 5, generator=G(12)).bfloat16()
    x[0] = 0.0
    x[1, 1, 2, 2] = float("nan")
    x[2, 0, 0, 0] = float("inf")
    x[3] = x[3] * 2.0 ** -130
    x[4] = x[4] * 2.0 ** 100
    x[5, 2, 4, 4] = -float("inf")
    e, x16 = tconv.scale_input(x.to(dev), 0)
    e_ref = O.conv_sample_exps(x, 0)
    assert e.cpu().numpy().tolist() == e_ref.tolist()
    assert _same_bits(x16, O.conv_scale_input(x, e_ref))


@pytest.mark.parametrize("layout", ["nchw", "channels_last"])
@pytest.mark.parametrize("O_,spatial", [(96, (7, 9)), (5, (3, 1)), (13, (1, 1)), (320, (24, 24))])
@pytest.mark.parametrize("with_bias", [False, True])
def test_conv_epilogue_matches_oracle(dev, layout, O_, spatial, with_bias):
    g = G(13)
    B = 3
    y16 = (torch.randn((B, O_) + spatial, generator=g) * 500).half()
    e = torch.tensor([-17, 2, 31], dtype=torch.int32)
    ws = torch.from_numpy(np.ldexp(np.float32(1), np.random.default_rng(1).integers(-20, 8, O_)).astype(np.float32))
    bias = (torch.randn(O_, generator=g) * 50).bfloat16() if with_bias else None
    yd = y16.to(dev)
    if layout == "channels_last":
        yd = yd.to(memory_format=torch.channels_last)
    out = tconv.unscale_output(yd, e.to(dev), ws.to(dev), None if bias is None else bias.to(dev))
    assert out.dtype == torch.bfloat16 and out.stride() == yd.stride()
    assert _same_bits(out.contiguous(), O.conv_epilogue(y16, e.numpy(), ws, bias))


# ---- tests/test_conv.py ----------------------------------------------------------------

def _check(dev, conv, shape, scale=1.0, channels_last=False, seed=0):
    conv = conv.to(dev).bfloat16()
    x = (torch.randn(shape, generator=G(seed)) * scale).bfloat16().to(dev)
    if channels_last:
        x = x.to(memory_format=torch.channels_last if x.dim() == 4 else torch.channels_last_3d)
    tc = convert_conv(copy.deepcopy(conv))
    with torch.no_grad():
        y = tc(x)
    r = O.conv_ref64(x.cpu(), tc.dequantized_weight().cpu(), None if tc.bias is None else tc.bias.detach().cpu(),
                     tc.stride, tc.padding, tc.dilation, tc.groups, tc.padding_mode,
                     tc._reversed_padding_repeated_twice)
    assert y.dtype == torch.bfloat16 and y.shape == r.shape and torch.isfinite(y).all()
    err = O.rel_err(y.cpu(), r)
    assert err < 3e-3, err
    return tc, x, y, err


CONV_CASES = [
    ("conv2d 3x3", lambda: nn.Conv2d(64, 96, 3, padding=1), (2, 64, 40, 56), False),
    ("conv2d 3x3 no bias stride 2", lambda: nn.Conv2d(64, 96, 3, stride=2, padding=1, bias=False), (2, 64, 40, 56),
     False),
    ("conv2d 3x3 channels_last", lambda: nn.Conv2d(64, 96, 3, padding=1), (2, 64, 40, 56), True),
    ("conv2d 3x3 reflect padding", lambda: nn.Conv2d(32, 32, 3, padding=1, padding_mode="reflect"), (1, 32, 33, 47),
     False),
    ("conv2d depthwise 5x5 channels_last", lambda: nn.Conv2d(96, 96, 5, padding=2, groups=96, bias=False),
     (1, 96, 16, 16), True),
    ("conv2d grouped 1x1", lambda: nn.Conv2d(96, 96, 1, groups=6, bias=False), (1, 96, 16, 16), False),
    ("conv2d 1x1 (scaled_linear path)", lambda: nn.Conv2d(128, 320, 1), (2, 128, 24, 24), False),
    ("conv2d 1x1 channels_last", lambda: nn.Conv2d(128, 320, 1), (2, 128, 24, 24), True),
    ("conv1d k=4", lambda: nn.Conv1d(48, 64, 4, padding=1), (3, 48, 100), False),
    ("conv3d 3x3x3", lambda: nn.Conv3d(32, 48, 3, padding=1), (1, 32, 5, 24, 40), False),
    ("conv3d 3x3x3 channels_last_3d", lambda: nn.Conv3d(32, 48, 3, padding=1), (1, 32, 5, 24, 40), True),
    ("conv2d 3x3 same padding, dilation 2", lambda: nn.Conv2d(16, 24, 3, padding="same", dilation=2),
     (2, 16, 19, 21), False),
    ("conv2d 3 input channels, odd sizes", lambda: nn.Conv2d(3, 8, 3, stride=2), (3, 3, 17, 15), False),
]


@pytest.mark.parametrize("name,make,shape,cl", CONV_CASES, ids=[c[0] for c in CONV_CASES])
def test_conv_cases(dev, name, make, shape, cl):
    torch.manual_seed(0)
    tc, x, y, err = _check(dev, make(), shape, channels_last=cl)
    if not tc._tbf16_plan.pointwise:
        # the scaled path is at most marginally worse than its CPU restatement
        # (the same arithmetic with the fp16 convolution's sum taken exactly)
        xin = x.cpu()
        if tc.padding_mode != "zeros":
            xin = F.pad(xin, tc._reversed_padding_repeated_twice, mode=tc.padding_mode)
        pad = 0 if tc.padding_mode != "zeros" else tc.padding
        emu = O.conv_forward(xin, tc.weight16.cpu(), tc.weight_scale.cpu(),
                             None if tc.bias is None else tc.bias.detach().cpu(), tc.stride, pad, tc.dilation,
                             tc.groups)
        r = O.conv_ref64(x.cpu(), tc.dequantized_weight().cpu(),
                         None if tc.bias is None else tc.bias.detach().cpu(), tc.stride, tc.padding, tc.dilation,
                         tc.groups, tc.padding_mode, tc._reversed_padding_repeated_twice)
        assert err <= 1.05 * O.rel_err(emu, r) + 1e-4, (err, O.rel_err(emu, r))


@pytest.mark.parametrize("scale", [3e4, 1e6, 1e-8])
def test_conv_scaled_inputs(dev, scale):
    """Inputs far outside fp16's range convert exactly (test_conv.py:58-60)."""
    torch.manual_seed(0)
    _check(dev, nn.Conv2d(64, 96, 3, padding=1), (2, 64, 40, 56), scale=scale, seed=1)
    _check(dev, nn.Conv3d(32, 48, 3, padding=1), (1, 32, 5, 24, 40), scale=scale, seed=2)


def test_conv_matches_reference_formula_on_gpu(dev):
    """The reference's own arithmetic (conv.py:49-60) in torch ops on the same GPU,
    with the same fp16 convolution call: the outputs agree bit for bit."""
    torch.manual_seed(0)
    conv = nn.Conv2d(64, 96, 3, padding=1).to(dev).bfloat16()
    x = (torch.randn(2, 64, 40, 56, generator=G(21)) * 5).bfloat16().to(dev)
    tc = convert_conv(copy.deepcopy(conv))
    with torch.no_grad():
        y = tc(x)
        amax = torch.linalg.vector_norm(x, float("inf"), dim=(1, 2, 3))
        e = torch.frexp(torch.where(amax.float() > 0, amax.float(), torch.ones_like(amax.float())))[1] \
            - tc._tbf16_plan.target_exp
        one = torch.ones_like(amax, dtype=torch.float32)
        x16 = torch.empty_like(x, dtype=torch.float16)
        torch.mul(x, torch.ldexp(one, -e).view(2, 1, 1, 1), out=x16)
        y16 = F.conv2d(x16, tc.weight16, None, tc.stride, tc.padding, tc.dilation, tc.groups)
        scale = (torch.ldexp(one, e)[:, None] * tc.weight_scale[None, :]).view(2, 96, 1, 1)
        ref = torch.empty_like(y16, dtype=torch.bfloat16)
        torch.addcmul(tc.bias.detach().view(1, 96, 1, 1), y16, scale, out=ref)
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


class CausalConv3d(nn.Conv3d):  # like diffusers' WanCausalConv3d: own forward, then super().forward
    def __init__(self, *a, **k):
        super().__init__(*a, **k)
        self._pad = (1, 1, 1, 1, 2, 0)
        self.padding = (0, 0, 0)

    def forward(self, x):
        return super().forward(F.pad(x, self._pad))


def test_conv_convert_nested_and_subclass(dev):
    """convert() reaches nested convs and subclasses, whose own forward still runs
    (test_conv.py:63-93); weight16 / weight_scale buffers replace the weight."""
    torch.manual_seed(0)
    model = nn.Sequential(nn.Conv2d(16, 32, 3, padding=1),
                          nn.Sequential(nn.SiLU(), nn.Conv2d(32, 16, 1))).to(dev).bfloat16()
    x = torch.randn(1, 16, 20, 20, generator=G(30)).bfloat16().to(dev)
    with torch.no_grad():
        r = copy.deepcopy(model).double()(x.double())
        tbf16.convert(model, sdpa=False, force=True)
        y = model(x)
    assert type(model[0]).__name__ == "TBF16Conv2d" and type(model[1][1]).__name__ == "TBF16Conv2d"
    assert model[0].weight is None and "0.weight16" in model.state_dict() and "0.weight_scale" in model.state_dict()
    assert O.rel_err(y.cpu(), r.cpu()) < 1e-2

    cc = CausalConv3d(8, 8, 3).to(dev).bfloat16()
    x = torch.randn(1, 8, 4, 10, 12, generator=G(31)).bfloat16().to(dev)
    with torch.no_grad():
        r = copy.deepcopy(cc).double()(x.double())
        m = nn.Sequential(cc)
        tbf16.convert(m, sdpa=False, force=True)
        y = m(x)
    assert type(m[0]).__name__ == "TBF16CausalConv3d"
    assert O.rel_err(y.cpu(), r.cpu()) < 1e-2
    # converting again changes nothing
    tbf16.convert(m, sdpa=False, force=True)
    assert type(m[0]).__name__ == "TBF16CausalConv3d"


def test_conv_native_paths_and_unbatched(dev):
    """Inputs that need gradients or are not bf16 run the native convolution on the
    dequantized weight (conv.py:36-38); an unbatched input is one sample."""
    torch.manual_seed(0)
    tc = convert_conv(nn.Conv2d(8, 12, 3, padding=1).to(dev).bfloat16())
    x = torch.randn(2, 8, 9, 9, generator=G(40)).bfloat16().to(dev)
    w = tc.dequantized_weight()
    xg = x.clone().requires_grad_()
    yg = tc(xg)
    assert torch.equal(yg, F.conv2d(x, w, tc.bias, 1, 1))
    yg.float().sum().backward()
    assert xg.grad is not None and xg.grad.shape == x.shape
    xf = x.float()
    with torch.no_grad():
        yf = tc(xf)
        assert yf.dtype == torch.float32
        assert torch.allclose(yf, F.conv2d(xf, w.float(), tc.bias.float(), 1, 1))
        y1 = tc(x[1])
        y2 = tc(x)
    # same exponent and scaled input as in the batch; the convolution may pick
    # another algorithm for one sample, so compare at bf16 resolution
    assert y1.shape == (12, 9, 9) and O.rel_err(y1.cpu(), y2[1].cpu()) < 1e-3
    with torch.no_grad():
        assert tc(x[:0]).shape == (0, 12, 9, 9)
    # helpers reject the wrong dtypes; samples with no elements take amax = 1
    with pytest.raises(TypeError):
        tconv.scale_input(x.half(), 0)
    e, x16 = tconv.scale_input(torch.empty(3, 0, 4, 4, dtype=torch.bfloat16, device=dev), -2)
    assert e.tolist() == [3, 3, 3] and x16.shape == (3, 0, 4, 4)
    with pytest.raises(TypeError):
        tconv.unscale_output(x, e, tc.weight_scale)
