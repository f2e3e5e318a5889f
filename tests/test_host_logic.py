"""Host-side control flow that needs no GPU: the attention-backward retry policy
(forced from the host with an injected attempt), routing thresholds, target
exponents and the conversion entry point's GPU check."""
import math
import warnings

import pytest
import torch
import torch.nn as nn

import importlib

import tbf16
from tbf16 import attention, autograd, ops

convert = importlib.import_module("tbf16.convert")  # the package rebinds `tbf16.convert` to the function
from oracle import tbf16_oracle as O


class _Fake:
    """Stands in for one backward attempt: overflows for the first `n_bad` calls."""

    def __init__(self, n_bad):
        self.n_bad, self.t_dos = n_bad, []

    def __call__(self, q, k, v, o16, lse, dout, exps, bias, scale, causal, t_do):
        self.t_dos.append(t_do)
        bad = len(self.t_dos) <= self.n_bad
        z = torch.zeros(1)
        # overflow word: float bits of the largest fp16 intermediate (+inf when overflowing)
        return z, z, z, torch.zeros(2, dtype=torch.int32), torch.tensor([0x7F800000 if bad else 0x46000000],
                                                                       dtype=torch.int32)


def _q(D):
    return torch.zeros(1, 1, 4, D)


@pytest.mark.parametrize("D", [64, 112, 128])
def test_retry_lowers_t_do_by_8(D):
    f = _Fake(2)
    autograd.attn_backward(_q(D), None, None, None, None, None, None, None, 1.0, False, check=True, attempt_fn=f)
    t0 = 12 - math.ceil(math.log2(D))
    assert f.t_dos == [t0, t0 - 8, t0 - 16]
    # same sequence as the oracle's restatement of autograd.py:177-189
    seq = []
    O.attn_bwd_retry(0, t0, lambda G: seq.append(G) or len(seq) <= 2)
    assert [t0 - g for g in seq] == [0, 8, 16] and seq[0] - seq[-1] == 16


def test_retry_gives_up_after_six():
    f = _Fake(100)
    with pytest.raises(FloatingPointError):
        autograd.attn_backward(_q(128), None, None, None, None, None, None, None, 1.0, False, check=True,
                               attempt_fn=f)
    assert len(f.t_dos) == autograd.ATTN_RETRIES == 6


def test_check_disabled_runs_once():
    f = _Fake(100)
    autograd.attn_backward(_q(128), None, None, None, None, None, None, None, 1.0, False, check=False, attempt_fn=f)
    assert f.t_dos == [5]


class _Done:
    """A finished CUDA event, for the deferred check of device-mode backwards."""

    def query(self):
        return True

    def synchronize(self):
        pass


class _Busy(_Done):
    def query(self):
        return False


def test_overflow_word_threshold():
    # 65504 (fp16 max) and 65519.99 round to finite fp16; 65520 and above do not
    for x, bad in ((65504.0, False), (65519.99, False), (65520.0, True), (1e30, True), (float("inf"), True),
                   (float("nan"), True), (0.0, False)):
        word = torch.tensor([x], dtype=torch.float32).view(torch.int32).abs()[0] if x == x else 0x7FC00000
        assert autograd._overflowed(int(word)) == bad, x


def test_deferred_check_raises_only_for_a_persistent_overflow():
    ok, inf, big = 0x46000000, 0x7F800000, 0x47800000  # 8192, +inf, 65536
    autograd._pending[:] = [(_Done(), torch.tensor([ok, inf], dtype=torch.int32)),   # retry not run: word 2 unused
                            (_Done(), torch.tensor([big, ok], dtype=torch.int32))]   # the retry fixed it
    autograd.check_pending()
    assert autograd._pending == []
    busy = (_Busy(), torch.tensor([inf, inf], dtype=torch.int32))
    autograd._pending[:] = [busy]
    autograd.check_pending()  # not finished: left for later, no error yet
    assert autograd._pending == [busy]
    with pytest.raises(FloatingPointError):
        autograd.check_pending(block=True)
    assert autograd._pending == []


def _sdpa_with_fake_kernels(monkeypatch, mode, persistent):
    """autograd.sdpa on CPU tensors with the kernel calls replaced: the forward returns
    zeros, the backward enqueues the overflow words of an attempt and its retry (both
    overflowing when `persistent`) as a device-mode backward does. Returns q's leaf."""
    monkeypatch.setattr(autograd, "CHECK_OVERFLOW", mode)

    def fwd(q, k, v, bias, is_causal, scale, v_exp, want_lse=False, want_o16=False, dropout_p=0.0, seed=0):
        z = torch.zeros_like(q)
        return z, torch.zeros(q.shape[:3]), z.half(), torch.zeros(2 + k.shape[0] * k.shape[1], dtype=torch.int32)

    def bwd(q, k, v, o16, lse, dout, exps, bias, sc, causal, dropout_p=0.0, seed=0, head_dim=None):
        words = [0x7F800000, 0x7F800000] if persistent else [0x7F800000, 0x46000000]
        autograd._pending.append((_Done(), torch.tensor(words, dtype=torch.int32)))
        return torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v), torch.zeros(2, dtype=torch.int32)

    monkeypatch.setattr(autograd.attention, "attn_forward", fwd)
    monkeypatch.setattr(autograd, "attn_backward", bwd)
    autograd._pending.clear()
    q, k, v = (torch.zeros(1, 2, 16, 64, dtype=torch.bfloat16, requires_grad=True) for _ in range(3))
    return q, autograd.sdpa(q, k, v, is_causal=True)


def test_device_mode_raises_from_the_same_backward(monkeypatch):
    """Device mode: an overflow that persists through the device-side retry raises
    FloatingPointError from the backward() call that produced it (an end-of-backward
    callback checks the words), as the reference's host loop raises inside backward
    (tbf16/autograd.py:184-189), so an optimizer step never sees those gradients.
    A retry that fixed the overflow raises nothing; the deferred mode leaves the
    error to check_pending()."""
    q, o = _sdpa_with_fake_kernels(monkeypatch, "device", persistent=True)
    with pytest.raises(FloatingPointError):
        o.float().sum().backward()
    assert autograd._pending == []
    q, o = _sdpa_with_fake_kernels(monkeypatch, "device", persistent=False)
    o.float().sum().backward()
    assert q.grad is not None and autograd._pending == []
    q, o = _sdpa_with_fake_kernels(monkeypatch, "deferred", persistent=True)
    o.float().sum().backward()
    assert len(autograd._pending) == 1
    with pytest.raises(FloatingPointError):
        autograd.check_pending(block=True)


def test_target_exp_matches_oracle():
    for K in (1, 7, 8, 100, 2048, 2560, 4096, 32768, 32769, 65536, 1 << 20):
        assert ops._target_exp(K) == O.target_exp(K)


def test_convert_without_gpu_warns_and_returns_model():
    m = nn.Sequential(nn.Linear(16, 16))
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        out = tbf16.convert(m)
    assert out is m and isinstance(m[0], nn.Linear) and type(m[0]) is nn.Linear
    assert any("MI355X" in str(x.message) for x in w)


def test_convert_train_swaps_class_only():
    m = nn.Sequential(nn.Linear(16, 16), nn.ReLU(), nn.Linear(16, 4))
    p0 = [id(p) for p in m.parameters()]
    tbf16.convert(m, train=True, sdpa=False, force=True)
    assert type(m[0]) is convert.TrainLinear and type(m[2]) is convert.TrainLinear
    assert [id(p) for p in m.parameters()] == p0


def test_shared_parameters_counts_each_module_once():
    """A weight tied between two modules is shared; a module reachable from two
    parents owns its weight once, so it is not treated as tied (the reference counts
    owners over the deduplicated module list, tbf16/convert.py:132-136)."""
    lin = nn.Linear(8, 8)
    twice = nn.ModuleDict({"a": nn.Sequential(lin), "b": nn.Sequential(lin)})
    assert convert._shared_parameters(twice) == set()
    emb, head = nn.Embedding(10, 8), nn.Linear(8, 10, bias=False)
    head.weight = emb.weight
    tied = nn.ModuleDict({"emb": emb, "head": head})
    assert convert._shared_parameters(tied) == {id(emb.weight)}


def test_mask_to_bias_shapes():
    keep = torch.ones(2, 7, dtype=torch.bool)
    keep[:, 5:] = False
    b = attention.mask_to_bias(keep[:, None, None, :], 2, 3, 4, 7, torch.device("cpu"))
    assert b.shape == (2, 3, 4, 7) and b.dtype == torch.float16 and b.stride(-1) == 1
    assert b.stride(1) == 0 and b.stride(2) == 0
    assert torch.isinf(b[:, :, :, 5:]).all() and (b[:, :, :, :5] == 0).all()
    add = torch.full((7,), -1e5)
    b2 = attention.mask_to_bias(add, 2, 3, 4, 7, torch.device("cpu"))
    assert torch.isinf(b2).all()  # large negatives become -inf in fp16, as the reference


def test_router_thresholds():
    assert convert.MIN_QUERY_ROWS == 16 and ops.FUSED_MIN_M == 256 and ops.SMALL_M == 2 and ops.L1_TARGET == 15
    # CPU tensors never take the tbf16 path
    q = torch.randn(1, 2, 32, 64).bfloat16()
    out = convert._sdpa(q, q, q)
    assert out.shape == q.shape


def test_public_api_names():
    for n in ["quantize_rows", "scaled_linear", "prepare_weight", "sdpa", "patch", "TuringBF16Mode", "convert",
              "Linear", "TrainLinear", "autograd", "install_sdpa", "uninstall_sdpa", "is_supported_gpu"]:
        assert hasattr(tbf16, n)
    for n in ["linear", "sdpa", "quantize_cols", "ScaledLinearFn", "ScaledSDPAFn", "FP32LinearFn"]:
        assert hasattr(tbf16.autograd, n)
    for n in ["_target_exp", "linear_q", "small_m_linear", "quantize_rows_shared"]:
        assert hasattr(tbf16.ops, n)
    for n in ["head_exp", "head_scale", "prepare_qkv", "expand_heads"]:
        assert hasattr(tbf16.attention, n)


def test_conv_module_host_logic():
    """tbf16.conv without a GPU: the public names of conv.py, convertible() only for
    bf16 GPU convs not yet converted, the generated TBF16<Conv> subclass keeps the
    native _conv_forward for the fallback path and is made once per class, and
    convert(force=True) leaves CPU convs alone."""
    from tbf16 import conv as tconv
    for n in ["convert_conv", "convertible", "scale_input", "unscale_output"]:
        assert hasattr(tconv, n)
    c2 = nn.Conv2d(4, 8, 3).bfloat16()
    assert not tconv.convertible(c2)  # on the CPU
    assert not tconv.convertible(nn.Linear(4, 4))
    cls = tconv._scaled_class(nn.Conv2d)
    assert cls.__name__ == "TBF16Conv2d" and issubclass(cls, nn.Conv2d)
    # the scaled forward sits in front of the native one, which stays reachable through super()
    assert cls.__mro__[1] is tconv.ScaledConvMixin and cls.__mro__[2] is nn.Conv2d
    assert tconv._scaled_class(nn.Conv2d) is cls
    m = nn.Sequential(nn.Conv2d(4, 8, 3).bfloat16(), nn.Conv1d(4, 4, 1).bfloat16())
    tbf16.convert(m, sdpa=False, force=True)
    assert type(m[0]) is nn.Conv2d and type(m[1]) is nn.Conv1d and m[0].weight is not None


def test_routing_predicate_shapes():
    """The one predicate convert(), patch() and tbf16.sdpa share: shapes the fused
    kernels do not compute (value head dim != key head dim, k/v shapes differ, GQA
    without enable_gqa, head dim > 256) are refused with a reason; head dims that are
    not a multiple of 8 are accepted (the caller zero-pads)."""
    from tbf16 import routing
    q = torch.zeros(2, 8, 32, 64)
    kv = torch.zeros(2, 8, 40, 64)
    assert routing.kernel_takes_qkv(q, kv, kv) is None
    assert routing.kernel_takes_qkv(q, kv, torch.zeros(2, 8, 40, 128)) is not None  # Dv != D
    assert routing.kernel_takes_qkv(q, kv, torch.zeros(2, 8, 41, 64)) is not None
    assert routing.kernel_takes_qkv(q, torch.zeros(1, 8, 40, 64), torch.zeros(1, 8, 40, 64)) is not None
    g = torch.zeros(2, 2, 40, 64)
    assert routing.kernel_takes_qkv(q, g, g) is not None
    assert routing.kernel_takes_qkv(q, g, g, enable_gqa=True) is None
    g3 = torch.zeros(2, 3, 40, 64)
    assert routing.kernel_takes_qkv(q, g3, g3, enable_gqa=True) is not None  # 8 % 3 != 0
    big = torch.zeros(1, 1, 32, 264)
    assert routing.kernel_takes_qkv(big, big, big) is not None
    odd = torch.zeros(1, 1, 32, 60)
    assert routing.kernel_takes_qkv(odd, odd, odd) is None
    # CPU tensors always stay native
    assert routing.attention_route(q.bfloat16(), kv.bfloat16(), kv.bfloat16()) == "native"
    with pytest.raises(ValueError):
        attention._check_qkv(q.bfloat16(), kv.bfloat16(), torch.zeros(2, 8, 40, 128).bfloat16(), False)


def test_routing_bind_sdpa():
    from tbf16 import routing
    q, k, v = object(), object(), object()
    c = routing.bind_sdpa((q, k), {"value": v, "is_causal": True})
    assert c["query"] is q and c["key"] is k and c["value"] is v and c["is_causal"] is True
    assert c["attn_mask"] is None and c["dropout_p"] == 0.0 and c["scale"] is None and c["enable_gqa"] is False
    c = routing.bind_sdpa((), {"query": q, "key": k, "value": v, "enable_gqa": True})
    assert c["enable_gqa"] is True
    with pytest.raises(TypeError):
        routing.bind_sdpa((q, k, v), {"query": q})
    with pytest.raises(TypeError):
        routing.bind_sdpa((q, k, v), {"bogus": 1})
    with pytest.raises(TypeError):
        routing.bind_sdpa((q, k), {})


def test_native_sdpa_hook_takes_dv_different_from_d():
    """A call torch accepts and the kernels do not (Dv != D) runs natively through the
    installed hook instead of raising."""
    q = torch.randn(1, 2, 32, 64).bfloat16()
    k = torch.randn(1, 2, 32, 64).bfloat16()
    v = torch.randn(1, 2, 32, 128).bfloat16()
    out = convert._sdpa(q, k, v)
    assert out.shape == (1, 2, 32, 128)


def test_tensor_memo_semantics():
    """TensorMemo: a hit needs the same live tensor at the same version; in-place
    changes rebuild; freed tensors drop their entries; capacity evicts the oldest."""
    import gc
    from tbf16 import routing
    memo = routing.TensorMemo(capacity=2)
    calls = []

    def build(tag):
        calls.append(tag)
        return tag

    a = torch.zeros(4)
    assert memo.get(a, "k", lambda: build("a1")) == "a1"
    assert memo.get(a, "k", lambda: build("a2")) == "a1"  # hit
    assert memo.get(a, "k2", lambda: build("a3")) == "a3"  # other key
    a.add_(1)  # version bump
    assert memo.get(a, "k", lambda: build("a4")) == "a4"
    b = torch.zeros(4)
    memo.get(b, "k", lambda: build("b1"))
    assert len(memo) <= 2
    n = len(memo)
    del b
    gc.collect()
    assert len(memo) == n - 1  # b's entry went with it
    assert calls == ["a1", "a3", "a4", "b1"]
