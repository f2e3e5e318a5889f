"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each check is chosen so that a plausible slip in the restatement (an off-by-one
in the exponent offset, a missing clamp, truncation instead of round-to-nearest,
a transposed operand, a dropped scale) fails: closed-form invariants,
torch's own RNE casts, an independent C restatement, brute force on tiny inputs
and fp64 references with closed-form special cases.
"""
import math

import numpy as np
import pytest
import torch

from oracle import pow2_c
from oracle import tbf16_oracle as O

ALL_BF16 = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
POS_BF16 = np.arange(0, 0x8000, dtype=np.uint32).astype(np.uint16)


def bf16_vals(bits):
    return O.bf16_bits_to_f32(bits)


@pytest.mark.parametrize("t", [-1, 0, 1, 5, 15])
def test_pow2_exp_invariant_on_every_normal_bf16(t):
    """amax * 2^p lands in [2^(t-1), 2^t) for every normal bf16 amax whose scale
    is not clamped (small_kernels.cu:11-18 comment)."""
    a = bf16_vals(POS_BF16)
    E = O.exp_field(a)
    p = O.pow2_exp(a, t)
    ok = (E >= 1) & (E <= 252) & (253 + t - E >= 1) & (253 + t - E <= 254)
    scaled = a[ok].astype(np.float64) * np.ldexp(1.0, p[ok].astype(np.int64))
    assert np.all(scaled >= 2.0 ** (t - 1)) and np.all(scaled < 2.0 ** t)
    # frexp identity for the same values: p = t - frexp_exp(amax)
    assert np.array_equal(p[ok], t - O.frexp_exp(a[ok]))


@pytest.mark.parametrize("t", [-1, 0, 15])
def test_pow2_exp_c_matches_numpy_all_patterns(t):
    a = bf16_vals(ALL_BF16)
    a = np.abs(a)
    for fused in (False, True):
        ref = O.pow2_exp_fused(a, t) if fused else O.pow2_exp(a, t)
        assert np.array_equal(pow2_c.pow2_exp(a, t, fused), ref)


def test_pow2_exp_edge_table():
    """Edge rows written out by hand from the clamps."""
    f = np.float32
    # zero row: e clamps to 1 -> se = clamp(252 + t, 1, 254)
    assert O.pow2_exp(f(0), 15) == 127 and O.pow2_exp(f(0), 0) == 125 and O.pow2_exp(f(0), -1) == 124
    # fused variant has the same upper clamp
    assert O.pow2_exp_fused(f(0), 15) == 127
    # amax = 1.0 (E = 127): s = 2^(t-1)
    for t in (-1, 0, 15):
        assert O.pow2_exp(f(1.0), t) == t - 1
    # huge amax: e clamps to 252 -> se = 1 + t (clamped to >= 1 in the small kernels)
    assert O.pow2_exp(f(np.inf), 0) == -126 and O.pow2_exp(f(np.inf), 15) == -111
    assert O.pow2_exp_fused(f(np.inf), -1) == -127   # no lower clamp: se = 0
    # the Triton variant overflows the scale for zero rows at t = 15 (documented divergence)
    assert O.pow2_exp_triton(f(0), 15) == 140


@pytest.mark.parametrize("p", [-126, -20, -1, 0, 3, 15, 29, 60, 127])
def test_scaled_f16_matches_torch_rne(p):
    """fp16(bf16 * 2^p): the C restatement, torch's RNE cast and the oracle agree
    on all 65,536 bf16 patterns (NaNs compared as NaN)."""
    x = bf16_vals(ALL_BF16)
    s = np.float32(np.ldexp(1.0, p))
    prod = (x * s).astype(np.float32)
    torch_bits = torch.from_numpy(prod).half().view(torch.int16).numpy().view(np.uint16)
    c_bits = pow2_c.scaled_f16_bits(ALL_BF16, p)
    nan_t = np.isnan(torch.from_numpy(torch_bits.view(np.int16)).view(torch.float16).float().numpy())
    nan_c = (c_bits & 0x7C00) == 0x7C00
    nan_c &= (c_bits & 0x3FF) != 0
    assert np.array_equal(nan_t, nan_c)
    assert np.array_equal(torch_bits[~nan_t], c_bits[~nan_t])


def test_f32_to_f16_exhaustive_sample():
    rng = np.random.default_rng(0)
    u = rng.integers(0, 1 << 32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32)
    x = x[np.isfinite(x)]
    tb = torch.from_numpy(x).half().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(pow2_c.f32_to_f16_bits(x), tb)


def test_f32_to_bf16_rne():
    rng = np.random.default_rng(1)
    u = rng.integers(0, 1 << 32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32)
    x = np.concatenate([x[np.isfinite(x)], np.array([0.0, -0.0, np.inf, -np.inf, 1.00390625, 1.01171875], np.float32)])
    tb = torch.from_numpy(x).bfloat16().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(pow2_c.f32_to_bf16_bits(x), tb)
    assert np.array_equal(O.f32_to_bf16_rne_bits(x), tb)


def _brute_quantize_rows(x, t, l1):
    """Pure-Python loop restatement of quantize_rows on a tiny input, using
    math.frexp for the exponent instead of exponent bits."""
    rows = []
    sinv = []
    for r in range(x.shape[0]):
        vals = [float(v) for v in x[r].float()]
        amax = sum(abs(v) for v in vals) if l1 else max([abs(v) for v in vals] + [0.0])
        amax = float(np.float32(amax))
        if amax == 0.0 or amax < 2.0 ** -126:
            e = 1 - 127 + 1  # E clamped to 1 -> frexp-style exponent of 2^-126 is -125
        else:
            e = math.frexp(amax)[1]
        p = max(-126, min(127, t - e))
        rows.append([v * 2.0 ** p for v in vals])
        sinv.append(2.0 ** -p)
    y = torch.tensor(rows, dtype=torch.float64).float().half()
    return y, torch.tensor(sinv, dtype=torch.float32)


@pytest.mark.parametrize("l1", [False, True])
@pytest.mark.parametrize("t", [0, 15])
def test_quantize_rows_brute_force(l1, t):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(6, 24, generator=g) * torch.tensor([1e-30, 1e-3, 1, 3e4, 1e20, 0.0])[:, None]
    x = x.bfloat16()
    y, s = O.quantize_rows(x, t, l1)
    yb, sb = _brute_quantize_rows(x, t, l1)
    assert torch.equal(y.view(torch.int16), yb.view(torch.int16))
    assert torch.equal(s, sb)
    # round trip: with the max at 2^14 nothing in these rows is an fp16 subnormal,
    # so y * s_inv reproduces x exactly
    if t == 15 and not l1:
        assert torch.equal((y[1:5].float() * s[1:5, None]).bfloat16(), x[1:5])


def test_quantize_cols_matches_rows_of_transpose():
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(40, 16, generator=g) * 7).bfloat16()
    yc, sc = O.quantize_cols(x, 0)
    yr, sr = O.quantize_rows(x.t().contiguous(), 0)
    assert torch.equal(yc.t().contiguous().view(torch.int16), yr.view(torch.int16))
    assert torch.equal(sc, sr)
    # row_mul: pow2 multipliers folded before the column amax
    rm = torch.ldexp(torch.ones(40), torch.randint(-5, 6, (40,), generator=g).float())
    yc2, sc2 = O.quantize_cols(x, -1, rm)
    xr = (x.float() * rm[:, None]).bfloat16()  # exact: pow2 multiples of bf16 values
    yr2, sr2 = O.quantize_rows(xr.t().contiguous(), -1)
    assert torch.equal(yc2.t().contiguous().view(torch.int16), yr2.view(torch.int16)) and torch.equal(sc2, sr2)


def test_target_exps():
    assert [O.target_exp(k) for k in (1, 8, 2048, 2560, 4096, 6144, 32768, 32769, 65536, 1 << 20)] == \
        [0, 0, 0, 0, 0, 0, 0, -1, -1, -3]
    # the bound the target is chosen for: K * 4^t <= 65504 (ops.py:30-31)
    for K in (2048, 32768, 40000, 1 << 20):
        assert K * 4.0 ** O.target_exp(K) <= 65536
    assert O.dw_target_exp(8192) == 0 and O.dw_target_exp(40000) == -1 and O.dw_target_exp(1 << 17) == -2
    assert O.attn_do_target(128) == 5 and O.attn_do_target(64) == 6 and O.attn_do_target(112) == 5


def test_linear_paths_vs_fp64():
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(64, 256, generator=g) * 3e4).bfloat16()
    w = (torch.randn(96, 256, generator=g) * 256 ** -0.5).bfloat16()
    b = torch.randn(96, generator=g).bfloat16()
    ref = O.linear_ref64(x, w, b)
    w16, ws = O.prepare_weight(w)
    for fn in (O.linear_fused, O.linear_small_m, O.linear_cublas_path):
        assert O.rel_err(fn(x, w16, ws, b), ref) < 3e-3
    # single rounding beats the double-rounding cuBLAS path emulation
    assert O.rel_err(O.linear_small_m(x, w16, ws, b), ref) <= O.rel_err(O.linear_cublas_path(x, w16, ws, b), ref)
    # GEMV
    assert O.rel_err(O.gemv(x[:1], w16, ws, b), O.linear_ref64(x[:1], w, b)) < 3e-3


def test_linear_exact_small_integers():
    """Small integers: every product and partial sum is exact in fp32 and the
    result is exactly representable in bf16, so the emulation must be bit-exact
    against integer arithmetic. A transposed operand or a dropped scale fails."""
    g = torch.Generator().manual_seed(6)
    x = torch.randint(-4, 5, (16, 32), generator=g).float()
    w = torch.randint(-3, 4, (24, 32), generator=g).float()
    x[3] = 0  # zero row -> 0 output
    y_int = (x.long() @ w.long().t()).float()
    xb, wb = x.bfloat16(), w.bfloat16()
    w16, ws = O.prepare_weight(wb)
    for fn in (O.linear_fused, O.linear_small_m):
        assert torch.equal(fn(xb, w16, ws).float(), y_int)
    assert torch.equal(O.scaled_linear(xb[:1], w16, ws).float(), y_int[:1])
    assert torch.equal(O.linear_fused(xb[:, :32], w16, ws)[3].float(), torch.zeros(24))


def test_head_exp_and_attn_exponents_brute_force():
    g = torch.Generator().manual_seed(7)
    q = (torch.randn(2, 3, 8, 16, generator=g) * torch.tensor([1, 100, 3e-5])[None, :, None, None]).bfloat16()
    k = (torch.randn(2, 3, 8, 16, generator=g) * 1e4).bfloat16()
    v = (torch.randn(2, 3, 8, 16, generator=g) * 2.0 ** -9).bfloat16()
    v[1, 2] = 0
    he = O.head_exp(q)
    for b in range(2):
        for h in range(3):
            am = max(abs(float(t)) for t in q[b, h].flatten())
            assert int(he[b, h]) == (math.frexp(am)[1] if am else 0)
    a, ev = O.attn_exponents(q, k, v, 13)
    eq = max(math.frexp(max(abs(float(t)) for t in q[b, h].flatten()))[1] for b in range(2) for h in range(3))
    ek = max(math.frexp(max(abs(float(t)) for t in k[b, h].flatten()))[1] for b in range(2) for h in range(3))
    a_ref = math.floor((ek - eq) / 2)
    a_ref = max(min(a_ref, 14 - eq), ek - 14)
    assert a == a_ref
    assert int(ev[1, 2]) == -13 and int(ev[0, 0]) == O.head_exp(v)[0, 0] - 13
    # scaled maxima stay below 2^14 in magnitude class (attention.py:42-43)
    assert eq + a <= 14 and ek - a <= 14 or (ek - eq) > 28


def _heads_with_exps(exps, S=4, D=8, seed=0):
    """(1, H, S, D) bf16 whose head h has max |x| = 0.75 * 2^exps[h] (frexp exponent
    exps[h]) and every other element smaller."""
    g = torch.Generator().manual_seed(seed)
    H = len(exps)
    x = torch.rand(1, H, S, D, generator=g) * 0.5
    x[0, :, 1, 2] = 0.75
    x = x * torch.ldexp(torch.ones(H), torch.tensor(exps, dtype=torch.float32))[None, :, None, None]
    return x.bfloat16()


@pytest.mark.parametrize("eq,ek", [(2, 7), (7, 2), (-3, 5), (5, -3), (0, 0), (-20, 9), (9, -20), (13, 14), (1, 27)])
def test_attn_exponent_a_balances_unclamped(eq, ek):
    """Without clamping (eq + ek <= 28) the split puts the scaled maxima' exponents
    eq + a and ek - a within one of each other, the key's side the larger one
    (floor, not ceil nor truncation toward zero: (7, 2) and (2, 7) both give 1),
    and neither above 2^14: every q.k product of the fp16 copies stays below 2^28."""
    q = _heads_with_exps([eq - 1, eq], seed=1)
    k = _heads_with_exps([ek, ek - 3], seed=2)
    v = _heads_with_exps([0, 0], seed=3)
    a, _ = O.attn_exponents(q, k, v, 13)
    assert 0 <= (ek - a) - (eq + a) <= 1
    assert eq + a <= 14 and ek - a <= 14
    # the scaled copies themselves: max exponents eq + a and ek - a, all values finite
    q16, k16, _, a2, _ = O.prepare_qkv(q, k, v, 13)
    assert a2 == a
    assert int(O.head_exp(q16).max()) == eq + a and int(O.head_exp(k16).max()) == ek - a
    assert float(q16.float().abs().max()) < 2.0 ** 14 and float(k16.float().abs().max()) < 2.0 ** 14


@pytest.mark.parametrize("eq,ek", [(10, 19), (14, 16), (15, 15), (20, 10), (30, 30), (40, -5), (-5, 40)])
def test_attn_exponent_a_key_clamp_decides(eq, ek):
    """eq + ek >= 29 (logits past the reference's stated 2^28 limit): the key's copy
    is put exactly at exponent 14 (a = ek - 14), also where the query's clamp
    14 - eq would bind first (eq + ek >= 30): the clamps' order makes the key's
    side win. The query's copy then exceeds 2^14 (or overflows fp16)."""
    q = _heads_with_exps([eq], seed=4)
    k = _heads_with_exps([ek], seed=5)
    v = _heads_with_exps([0], seed=6)
    a, _ = O.attn_exponents(q, k, v, 0)
    assert ek - a == 14
    assert eq + a >= 15
    if eq + ek >= 30:  # the case covers the query's clamp binding first
        assert 14 - eq < math.floor((ek - eq) / 2)


def test_attn_exponent_a_boundary_28_29():
    """At eq + ek = 28 the balanced split still fits (both <= 14); one more and the
    key's clamp takes over."""
    for eq in range(-10, 30):
        ek = 28 - eq
        a, _ = O.attn_exponents(_heads_with_exps([eq]), _heads_with_exps([ek]), _heads_with_exps([0]), 0)
        assert eq + a <= 14 and ek - a <= 14 and 0 <= (ek - a) - (eq + a) <= 1
        a1, _ = O.attn_exponents(_heads_with_exps([eq]), _heads_with_exps([ek + 1]), _heads_with_exps([0]), 0)
        assert ek + 1 - a1 == 14


def test_reference_attention_arith_pins():
    """The emulation of the reference's inference arithmetic: within fp16/bf16 error
    of fp64 on peaky scaled heads; q = 0 gives the causal prefix means of V up to
    the output roundings; its only difference from this build's arithmetic
    (sdpa_fp16_emulated) is the fp16 rounding of O / l, so the two differ by at most
    one fp16 rounding plus one bf16 ulp per element, and are identical where O / l is
    exactly an fp16 value (one-hot rows copying a V row)."""
    g = torch.Generator().manual_seed(21)
    q = (torch.randn(1, 2, 48, 32, generator=g) * 2.0 ** 9).bfloat16()
    k = (torch.randn(1, 2, 48, 32, generator=g) * 2.0 ** 8).bfloat16()
    v = (torch.randn(1, 2, 48, 32, generator=g) * 2.0 ** 11).bfloat16()
    ref = O.sdpa_ref64(q, k, v, causal=True)
    r = O.sdpa_reference_arith(q, k, v, causal=True)
    assert r.dtype == torch.bfloat16 and O.rel_err(r, ref) < 3e-3
    mine, _, _ = O.sdpa_fp16_emulated(q, k, v, causal=True)
    d = (r.double() - mine.double()).abs()
    bound = mine.double().abs() * (2.0 ** -11 + 2.0 ** -7) + 1e-30
    assert bool((d <= bound).all())
    qz = torch.zeros_like(q)
    rz = O.sdpa_reference_arith(qz, k, v, causal=True)
    prefix = torch.cumsum(v.double(), 2) / torch.arange(1, 49, dtype=torch.float64)[:, None]
    assert O.rel_err(rz, prefix) < 3e-3
    # one-hot rows: P is exactly 1 on one key, O / l a bf16 V row, no rounding at all
    S, D = 16, 16
    qq = torch.zeros(1, 1, S, D)
    for i in range(S):
        qq[0, 0, i, i] = 64.0
    vv = torch.randn(1, 1, S, D, generator=g).bfloat16()
    ro = O.sdpa_reference_arith(qq.bfloat16(), qq.bfloat16(), vv, causal=False)
    assert torch.equal(ro, vv)


def test_reference_attention_bwd_arith_pins():
    """The emulation of the reference's training attention: exponents equal the
    closed forms (attn_exponents with v_exp = 0, attn_bwd_exponents); output and
    gradients within fp16-level error of fp64 autograd, with GQA (the fp32 group
    sum) and without."""
    g = torch.Generator().manual_seed(22)
    for H, Hkv in ((2, 2), (4, 2)):
        q = (torch.randn(1, H, 40, 32, generator=g) * 3).bfloat16()
        k = (torch.randn(1, Hkv, 40, 32, generator=g) * 3).bfloat16()
        v = (torch.randn(1, Hkv, 40, 32, generator=g) * 2.0 ** 10).bfloat16()
        do = (torch.randn(1, H, 40, 32, generator=g) * 2.0 ** -20).bfloat16()
        o, dq, dk, dv, (a, ev, e, G) = O.sdpa_bwd_reference_arith(q, k, v, do, causal=True)
        a0, ev0 = O.attn_exponents(q, k, v, 0)
        e0, _, G0 = O.attn_bwd_exponents(do, O.expand_heads(ev0, H), 32)
        assert (a, e, G) == (a0, e0, G0) and torch.equal(ev, ev0)
        ro, rdq, rdk, rdv = O.sdpa_grads_ref64(q, k, v, do, causal=True)
        for got, want in ((o, ro), (dq, rdq), (dk, rdk), (dv, rdv)):
            assert torch.isfinite(got).all() and O.rel_err(got, want) < 5e-3


def test_attention_closed_forms():
    """q = 0: uniform softmax, so row i of a causal output is the mean of V rows
    0..i. One-hot peaky logits copy one V row."""
    g = torch.Generator().manual_seed(8)
    S, D = 32, 16
    v = torch.randn(1, 2, S, D, generator=g).bfloat16()
    k = torch.randn(1, 2, S, D, generator=g).bfloat16()
    q = torch.zeros(1, 2, S, D).bfloat16()
    o = O.sdpa_ref64(q, k, v, causal=True)
    prefix = torch.cumsum(v.double(), 2) / torch.arange(1, S + 1, dtype=torch.float64)[:, None]
    assert torch.allclose(o, prefix, atol=1e-12)
    o16, _, _ = O.sdpa_fp16_emulated(q, k, v, causal=True)
    assert O.rel_err(o16, prefix) < 3e-3
    # one-hot: k = e_j * big, q = e_j -> query attends to the key sharing its one-hot
    kk = torch.zeros(1, 1, S, D)
    qq = torch.zeros(1, 1, S, D)
    for i in range(S):
        kk[0, 0, i, i % D] = 60.0
        qq[0, 0, i, i % D] = 60.0
    kk[0, 0, D:] = 0
    vv = torch.randn(1, 1, S, D, generator=g)
    o = O.sdpa_ref64(qq.bfloat16(), kk.bfloat16(), vv.bfloat16(), causal=False)
    assert torch.allclose(o[0, 0, :D], vv.bfloat16().double()[0, 0, :D], atol=1e-6)


def test_attention_emulation_vs_fp64_scaled_heads():
    g = torch.Generator().manual_seed(9)
    q = (torch.randn(1, 2, 64, 32, generator=g) * 2.0 ** 9).bfloat16()
    k = (torch.randn(1, 2, 64, 32, generator=g) * 2.0 ** 8).bfloat16()
    v = (torch.randn(1, 2, 64, 32, generator=g) * 2.0 ** 11).bfloat16()
    ref = O.sdpa_ref64(q, k, v, causal=True)
    out, a, ev = O.sdpa_fp16_emulated(q, k, v, causal=True)
    assert O.rel_err(out, ref) < 3e-3
    # unscaled fp16 logits would overflow: the 2^a / 2^-a split is doing work
    assert not torch.isfinite((q.half() @ k.half().transpose(-1, -2))).all()


def test_attn_bwd_exponents_and_retry():
    do = (torch.randn(1, 2, 8, 128) * 2.0 ** -20).bfloat16()
    ev_q = torch.tensor([[3, -2]], dtype=torch.int32)
    e, t_do, G = O.attn_bwd_exponents(do, ev_q, 128)
    he = O.head_exp(do)
    assert e == int(max(he[0, 0] + 3, he[0, 1] - 2)) and t_do == 5 and G == 5 - e
    # overflow on the first two attempts -> G drops by 8 twice
    calls = []
    G_acc = O.attn_bwd_retry(e, t_do, lambda g_: calls.append(g_) or len(calls) <= 2)
    assert calls == [G, G - 8, G - 16] and G_acc == G - 16
    with pytest.raises(FloatingPointError):
        O.attn_bwd_retry(e, t_do, lambda g_: True)


def _g_by_search(dout, ev_q, t_do):
    """The G the reference's backward picks, found from what it is for
    (autograd.py:173-176: "scale [dO 2^ev] by g = 2^G so its max sits at 2^t_do"):
    the one integer G for which the largest math.frexp exponent of the scaled head
    maxima amax|dO[b,h]| 2^(ev_q[b,h] + G) is t_do, searched over a wide range in
    fp64. Heads of zeros scale to zero and take no part."""
    amax = dout.double().abs().amax(dim=(-2, -1))
    found = [G for G in range(-400, 400)
             if max(math.frexp(math.ldexp(float(amax[b, h]), int(ev_q[b, h]) + G))[1]
                    for b in range(amax.shape[0]) for h in range(amax.shape[1]) if amax[b, h] > 0) == t_do]
    assert len(found) == 1
    return found[0]


def test_attn_bwd_exponents_put_the_scaled_max_at_t_do():
    """attn_bwd_exponents against the reference's stated purpose: the largest scaled
    dO head maximum lands in [2^(t_do - 1), 2^t_do) and no head exceeds it, for
    per-head magnitudes across the exponent range, negative ev, and GQA (ev_q =
    expand_heads(ev), each query head using kv head h // (H / Hkv))."""
    g = torch.Generator().manual_seed(40)
    for trial in range(12):
        B, Hkv, group = 1 + trial % 2, 1 + trial % 3, 1 + trial % 4
        H = Hkv * group
        mags = torch.randint(-30, 20, (B, H, 1, 1), generator=g).double()
        do = (torch.randn(B, H, 5, 16, generator=g).double() * torch.exp2(mags)).bfloat16()
        ev = torch.randint(-12, 14, (B, Hkv), generator=g, dtype=torch.int32)
        ev_q = O.expand_heads(ev, H)
        for b in range(B):
            for h in range(H):
                assert int(ev_q[b, h]) == int(ev[b, h // group])
        for D in (64, 128, 256):
            e, t_do, G = O.attn_bwd_exponents(do, ev_q, D)
            assert t_do == 12 - math.ceil(math.log2(D)) and G == t_do - e
            assert G == _g_by_search(do, ev_q, t_do), (trial, D)
            amax = do.double().abs().amax(dim=(-2, -1)) * torch.exp2((ev_q + G).double())
            assert float(amax.max()) >= 2.0 ** (t_do - 1) and float(amax.max()) < 2.0 ** t_do


def test_attn_bwd_exponents_zero_head_enters_through_ev():
    """A head of dO that is all zeros has head_exp 0 ("0 for all-zero heads",
    attention.py:25), so it enters e through its ev_q alone (autograd.py:175), as a
    head whose maximum were in [0.5, 1): hand-derived cases at D = 128 (t_do = 5).
    Head 0 is zero, head 1 has amax 3 (frexp exponent 2)."""
    do = torch.zeros(1, 2, 4, 8)
    do[0, 1, 2, 3] = -3.0
    do = do.bfloat16()
    # ev_q = (7, 2): the zero head decides, e = max(0 + 7, 2 + 2) = 7, G = 5 - 7 = -2;
    # the non-zero head then scales to 3 * 2^(2 - 2) = 3 < 2^4: below t_do
    e, t_do, G = O.attn_bwd_exponents(do, torch.tensor([[7, 2]], dtype=torch.int32), 128)
    assert (e, t_do, G) == (7, 5, -2)
    # ev_q = (3, 2): the non-zero head decides, e = 4, G = 1, 3 * 2^3 = 24 in [16, 32)
    e, t_do, G = O.attn_bwd_exponents(do, torch.tensor([[3, 2]], dtype=torch.int32), 128)
    assert (e, t_do, G) == (4, 5, 1) and G == _g_by_search(do, torch.tensor([[3, 2]]), 5)
    # the zero head acts exactly like a head of constant 0.75 (frexp exponent 0)
    stand_in = do.clone()
    stand_in[0, 0] = 0.75
    for ev_q in ([[7, 2]], [[3, 2]], [[-5, 0]], [[4, 2]]):
        evq = torch.tensor(ev_q, dtype=torch.int32)
        assert O.attn_bwd_exponents(do, evq, 128) == O.attn_bwd_exponents(stand_in, evq, 128)
    # all heads zero: e = max(ev_q)
    assert O.attn_bwd_exponents(torch.zeros(1, 3, 2, 8).bfloat16(),
                                torch.tensor([[-4, -9, -6]], dtype=torch.int32), 64) == (-4, 6, 10)


def _dominant_key(S, D, do_signs):
    """Key 0 takes ~99% of every query's attention (logit 12.5 against 0) and each
    query head's dO is a constant +-1, so dO16 = 2^(t_do - 1) = 32 at D = 64 and
    dv16 of key 0 is S * P * 32 per query head, with sign do_signs[h] (one kv head)."""
    H = len(do_signs)
    q = torch.zeros(1, H, S, D)
    q[..., 0] = 10.0
    k = torch.zeros(1, 1, S, D)
    k[0, 0, 0, 0] = 10.0
    v = torch.randn(1, 1, S, D, generator=torch.Generator().manual_seed(31))
    do = torch.ones(1, H, S, D) * torch.tensor(do_signs, dtype=torch.float32)[None, :, None, None]
    return tuple(t.bfloat16() for t in (q, k, v, do))


@pytest.mark.parametrize("S,signs,retries", [(1536, (1, 1), 0), (2304, (1, -1), 1), (2304, (1,), 1),
                                             (1536, (1,), 0)])
def test_reference_bwd_retry_checks_each_query_head(S, signs, retries):
    """The emulation retries on each query head's fp16 gradient, before the GQA group
    sum: dv16 of key 0 is S * P * 32 with P = e^12.5 / (e^12.5 + S - 1) (logit
    12.5 against S - 1 zeros). At S = 1536 each head's 48.9k fits fp16 while two
    heads sum to 97.7k (no retry); at S = 2304 each head's 73.1k overflows while a
    +1 and a -1 head cancel (one retry, G lowered by 8)."""
    p0 = math.exp(12.5) / (math.exp(12.5) + S - 1)
    assert (S * p0 * 32 >= 65520) == (retries == 1)
    q, k, v, do = _dominant_key(S, 64, signs)
    _, _, _, dv, (a, ev, e, G) = O.sdpa_bwd_reference_arith(q, k, v, do, causal=False)
    e0, t_do, G0 = O.attn_bwd_exponents(do, O.expand_heads(ev, len(signs)), 64)
    assert e == e0 and G == G0 - 8 * retries
    want = sum(signs) * S * p0  # dv of key 0 per element of dO's constant row
    assert torch.isfinite(dv).all() and abs(float(dv[0, 0, 0, 0]) - want) <= 0.01 * abs(want) + 1e-3


def test_ref64_attn_bwd64_matches_autograd_reference():
    """tests/_ref64.attn_bwd64 (the hand-written fp64 gradient the GPU tests hold
    configs[4] against) equals the finite-difference-pinned fp64 autograd of
    O.sdpa_grads_ref64, causal and not, with GQA (summed per kv head)."""
    from _ref64 import attn_bwd64
    g = torch.Generator().manual_seed(41)
    for H, Hkv, causal in ((2, 2, True), (4, 2, True), (3, 1, False)):
        q = torch.randn(2, H, 9, 8, generator=g).double()
        k = torch.randn(2, Hkv, 9, 8, generator=g).double()
        v = torch.randn(2, Hkv, 9, 8, generator=g).double()
        do = torch.randn(2, H, 9, 8, generator=g).double()
        o, dq, dk, dv = attn_bwd64(q, k, v, do, causal)
        ke, ve = O.expand_heads(k, H), O.expand_heads(v, H)
        ro, rdq, rdk, rdv = O.sdpa_grads_ref64(q, ke, ve, do, causal=causal)
        rdk = rdk.view(2, Hkv, H // Hkv, 9, 8).sum(2)
        rdv = rdv.view(2, Hkv, H // Hkv, 9, 8).sum(2)
        for a, b in ((o, ro), (dq, rdq), (dk, rdk), (dv, rdv)):
            assert torch.allclose(a, b, rtol=1e-10, atol=1e-12)


def test_attention_grads_fp64_against_finite_difference():
    """The fp64 autograd reference itself: a directional finite difference."""
    g = torch.Generator().manual_seed(10)
    q, k, v = (torch.randn(1, 1, 6, 4, generator=g).double() for _ in range(3))
    do = torch.randn(1, 1, 6, 4, generator=g).double()
    o, dq, dk, dv = O.sdpa_grads_ref64(q, k, v, do, causal=True)
    eps = 1e-6
    for t, gt in ((q, dq), (k, dk), (v, dv)):
        d = torch.randn(t.shape, generator=g).double()
        args = [q, k, v]
        i = [id(q), id(k), id(v)].index(id(t))
        ap, am = list(args), list(args)
        ap[i] = t + eps * d
        am[i] = t - eps * d
        fd = ((O.sdpa_ref64(*ap, causal=True) - O.sdpa_ref64(*am, causal=True)) * do).sum() / (2 * eps)
        assert abs(float(fd) - float((gt * d).sum())) < 1e-6


def test_linear_train_bwd_vs_fp64():
    g = torch.Generator().manual_seed(11)
    M, K, N = 96, 64, 80
    x = (torch.randn(M, K, generator=g) * 1e4).bfloat16()
    w = (torch.randn(N, K, generator=g) * K ** -0.5).bfloat16()
    dy = (torch.randn(M, N, generator=g) * 1e-8).bfloat16()
    y, x16, sx, w16, sw = O.linear_train_fwd(x, w)
    dx, dw, db, _ = O.linear_train_bwd(dy, x16, sx, w)
    assert O.rel_err(y, O.linear_ref64(x, w)) < 3e-3
    assert O.rel_err(dx, dy.double() @ w.double()) < 3e-3
    assert O.rel_err(dw, dy.double().t() @ x.double()) < 3e-3
    assert O.rel_err(db.float(), dy.double().sum(0)) < 3e-3


def test_dropout_mask_pins():
    """fmix32: the published finalizer value fmix32(1) = 0x514e28b7, a scalar
    pure-Python restatement, bijectivity on a 2^20 sample; the keep rule: exact
    thresholds, keep rates within 5 sigma, element-wise scalar restatement."""
    assert int(O.fmix32(1)) == 0x514E28B7 and int(O.fmix32(0)) == 0

    def fm(h):
        h &= 0xFFFFFFFF
        h ^= h >> 16
        h = (h * 0x85EBCA6B) & 0xFFFFFFFF
        h ^= h >> 13
        h = (h * 0xC2B2AE35) & 0xFFFFFFFF
        return h ^ (h >> 16)

    xs = np.random.default_rng(0).integers(0, 1 << 32, 3000, dtype=np.uint64)
    assert [int(v) for v in O.fmix32(xs)] == [fm(int(x)) for x in xs]
    assert len(np.unique(O.fmix32(np.arange(1 << 20)))) == 1 << 20

    assert O.dropout_params(0.0)[0] == 0
    thr, sc = O.dropout_params(0.25)
    assert thr == 16384 and sc == np.float32(1.0) / np.float32(0.75)
    assert O.dropout_params(1e-9)[0] == 1 and O.dropout_params(0.9999999)[0] == 65535

    seed = 0x0123_4567_89AB_CDEF
    for p in (0.1, 0.5, 0.9):
        m = O.dropout_keep(seed, 5, 1024, np.arange(1024), np.arange(1024), p)
        keep = 1.0 - O.dropout_params(p)[0] / 65536.0
        sigma = math.sqrt(keep * (1 - keep) / m.size)
        assert abs(m.mean() - keep) < 5 * sigma, (p, m.mean(), keep)

    lo, hi = seed & 0xFFFFFFFF, seed >> 32
    thr, _ = O.dropout_params(0.3)
    m = O.dropout_keep(seed, 7, 100, np.arange(100), np.arange(64), 0.3)
    for qi in (0, 1, 57, 99):
        row = fm(((7 * 100 + qi) & 0xFFFFFFFF) ^ lo)
        for kk in (0, 1, 2, 33, 63):
            u = fm((row + (kk >> 1) * 0x9E3779B9 + hi) & 0xFFFFFFFF)
            half = (u >> 16) if kk & 1 else (u & 0xFFFF)
            assert bool(m[qi, kk]) == (half >= thr)


# ---- scaled convolutions (tbf16/conv.py) --------------------------------------------

def _bf16_from_bits(bits, shape):
    return torch.from_numpy(np.asarray(bits, dtype=np.uint16).astype(np.int16)).view(torch.bfloat16).reshape(shape)


@pytest.mark.parametrize("t", [-3, -1, 0])
def test_conv_sample_exps_pins(t):
    """Every positive bf16 as a sample's max: normal maxima land in [2^(t-1), 2^t)
    after scaling by 2^-e; subnormal maxima match math.frexp; zero and NaN samples
    take amax = 1, infinite ones frexp's 0 (conv.py:28-31,49-50)."""
    mags = POS_BF16[:0x7F80]  # +0 ... largest finite
    x = _bf16_from_bits(mags, (len(mags), 1))
    x = torch.cat([x, -x[:, :1] * 0.5], dim=1)  # second element smaller, negative
    e = O.conv_sample_exps(x, t)
    a = bf16_vals(mags).astype(np.float64)
    normal = (mags >= 0x0080)
    scaled = a[normal] * np.ldexp(1.0, -e[normal].astype(np.int64))
    assert np.all(scaled >= 2.0 ** (t - 1)) and np.all(scaled < 2.0 ** t)
    sub = np.nonzero((mags > 0) & ~normal)[0]
    assert all(e[i] == math.frexp(float(a[i]))[1] - t for i in sub)
    assert e[0] == 1 - t  # all-zero sample
    special = _bf16_from_bits([0x7F80, 0x0000, 0x7FC0, 0x3F80, 0xFF80, 0x3F80], (3, 2))
    assert O.conv_sample_exps(special, t).tolist() == [-t, 1 - t, -t]  # inf; NaN -> 1 - t; -inf
    assert O.conv_sample_exps(_bf16_from_bits([0x7FC0, 0x4000], (1, 2)), t).tolist() == [1 - t]


def test_conv_scale_input_exact_and_rne():
    """x16 * 2^e reproduces x exactly for elements inside fp16's normal range, and
    every element equals torch's RNE cast of the fp32 product."""
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(3, 5, 7, 9, generator=g) * torch.tensor([1e-6, 1.0, 3e4]).view(3, 1, 1, 1)).bfloat16()
    x[1, 0, 0, :4] = 0.0
    x[2, 1, 2, 3] = 2e-3  # > 2^14 below the sample max: an fp16 subnormal
    e = O.conv_sample_exps(x, 0)
    x16 = O.conv_scale_input(x, e)
    back = x16.double() * torch.from_numpy(np.ldexp(1.0, e.astype(np.int64))).view(3, 1, 1, 1)
    normal = x16.float().abs() >= 2.0 ** -14
    assert torch.equal(back[normal], x.double()[normal])
    assert x16.float().abs().amax() < 1.0 and x16.float().abs().amax() >= 0.5  # t = 0: [2^-1, 2^0)
    for b in range(3):
        ref = (x[b].float() * float(np.ldexp(np.float32(1), -int(e[b])))).half()
        assert torch.equal(x16[b].view(torch.int16), ref.view(torch.int16))


def test_conv_epilogue_bits():
    """conv_epilogue against a numpy restatement at bit level: exact product in
    fp64, one rounding to fp32 after the bias add, then RNE to bf16."""
    g = torch.Generator().manual_seed(4)
    B, O_, P = 3, 5, 11
    y16 = (torch.randn(B, O_, P, generator=g) * 300).half()
    e = np.array([-20, 3, 40], dtype=np.int32)
    ws = torch.from_numpy(np.ldexp(np.float32(1), np.array([-7, 0, 5, -30, 2])).astype(np.float32))
    bias = (torch.randn(O_, generator=g) * 100).bfloat16()
    for bb in (None, bias):
        out = O.conv_epilogue(y16, e, ws, bb)
        ex = (y16.double().numpy() * np.ldexp(1.0, e.astype(np.int64))[:, None, None]
              * ws.double().numpy()[None, :, None])
        if bb is not None:
            ex = ex + bb.double().numpy()[None, :, None]
        ref_bits = O.f32_to_bf16_rne_bits(ex.astype(np.float32))
        assert np.array_equal(out.view(torch.int16).numpy().astype(np.uint16), ref_bits)


def test_conv_forward_exact_integers_and_fp64_bar():
    """Small-integer inputs and weights: every stage is exact, so the restatement
    equals the fp64 convolution rounded once to bf16. Random inputs: the reference's
    bar of 3e-3 (tests/test_conv.py:43), and a transposed weight fails it."""
    g = torch.Generator().manual_seed(5)
    x = torch.randint(-4, 5, (2, 6, 9, 8), generator=g).bfloat16()
    w = torch.randint(-3, 4, (7, 6, 3, 3), generator=g).bfloat16()
    bias = torch.randint(-8, 9, (7,), generator=g).bfloat16()
    w16, ws = O.conv_weight(w)
    assert torch.equal((w16.float() * ws.view(-1, 1, 1, 1)).bfloat16(), w)
    y = O.conv_forward(x, w16, ws, bias, 1, 1)
    assert torch.equal(y, O.conv_ref64(x, w, bias, 1, 1).bfloat16())
    x = (torch.randn(2, 16, 12, 10, generator=g) * 7).bfloat16()
    w = (torch.randn(24, 16, 3, 3, generator=g) * 0.1).bfloat16()
    w16, ws = O.conv_weight(w)
    r = O.conv_ref64(x, w, None, 2, 1)
    assert O.rel_err(O.conv_forward(x, w16, ws, None, 2, 1), r) < 3e-3
    w16t = w16.transpose(2, 3).contiguous()
    assert O.rel_err(O.conv_forward(x, w16t, ws, None, 2, 1), r) > 0.1
