"""CPU restatement of tbf16's scaled-fp16 hot path.

TEST INFRASTRUCTURE ONLY. This module is the checker for the HIP kernels: only
`tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may
import it. The product package (`turing-bf16_amd/tbf16`) never imports it and has
no CPU fallback.

Every function cites the reference line it restates (paths relative to the
tech-cosmos/turing-bf16 tree). Bit-level parts (exponents, fp16/bf16 payloads) are
exact; floating-point GEMM/attention parts run in fp32 (the reference's
accumulation type) or fp64 (the accuracy reference the reference's tests use).

How each function is pinned (checked by tests/test_oracle.py):
  pow2_exp / pow2_exp_fused   closed-form invariant amax*2^p in [2^(t-1), 2^t) for
                              every normal bf16 amax, frexp identity, edge table,
                              the C restatement (oracle/pow2.c) compared on all
                              65,536 bf16 patterns at test time (no stored KAT file:
                              the reference ships none).
  quantize_rows/quantize_cols payload == torch's RNE float->half of the same fp32
                              product; s_inv*scale == 1; brute force on tiny inputs.
  bf16/fp16 rounding          torch CPU RNE casts (library routines) and pow2.c.
  linear_fused / gemv /       fp64 matmul of the same bf16 values (rel err bound),
  linear_cublas_path          exact small-integer cases where fp32 is exact.
  attn_exponents / head_exp   torch.frexp on amax; brute-force loop over heads; a's
                              floor and both clamps by the invariants they exist for
                              (balanced scaled maxima, each at most 2^14, the key's
                              clamp winning when both bind).
  sdpa_reference_arith /      fp64 softmax attention within fp16-level error; the
  sdpa_bwd_reference_arith    closed forms (q = 0 -> prefix means, one-hot copy);
                              fp64 autograd gradients within fp16-level error; every
                              output rounding they model checked on its own.
  sdpa_ref64 / attn_*         closed forms: q=0 -> prefix mean of V rows, one-hot
                              logits copy a V row; fp64 autograd for gradients.
  attn_bwd_exponents / retry  the purpose autograd.py:173-176 states: the G found
                              by searching for the one that puts the largest scaled
                              dO head maximum at 2^t_do (fp64, math.frexp), with
                              GQA-expanded and negative ev; hand-derived cases where
                              an all-zero dO head enters e through ev_q; the retry
                              sequence with an injected overflowing backward; the
                              per-query-head overflow check of the emulation on
                              dominant-key cases whose dv16 is known in closed form
                              (per head vs group sum disagreeing both ways).
  fmix32 / dropout_keep       this build's own dropout mask (the reference draws its
                              mask from torch's Philox stream, not comparable bit for
                              bit): the published finalizer value fmix32(1) =
                              0x514e28b7, a scalar pure-Python restatement, the
                              finalizer's bijectivity on samples, keep rates.
  conv_sample_exps            amax * 2^-e in [2^(t-1), 2^t) for every normal bf16
                              amax, math.frexp brute force over bf16 subnormal
                              maxima, the zero / NaN / inf cases of conv.py:28-31.
  conv_scale_input            x16 * 2^e == x exactly for elements within fp16's
                              normal range; torch's RNE cast elsewhere.
  conv_epilogue               an fp64 -> fp32 -> bf16 numpy restatement (bit level).
  conv_forward / conv_ref64   exact small-integer convolutions; fp64 rel err bar
                              of tests/test_conv.py:43 on random inputs.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

FP16_MAX = 65504.0
# Smallest |x| that rounds to inf in fp16 (round-to-nearest-even).
FP16_OVERFLOW = 65520.0


# ---------------------------------------------------------------------------
# A1 / A2: power-of-two exponents (integer arithmetic on fp32 exponent bits)
# ---------------------------------------------------------------------------

def exp_field(amax) -> np.ndarray:
    """Biased fp32 exponent field (bits >> 23) & 0xFF of float32 values."""
    a = np.ascontiguousarray(np.asarray(amax, dtype=np.float32))
    return ((a.view(np.int32) >> 23) & 0xFF).astype(np.int64)


def pow2_exp(amax, t: int) -> np.ndarray:
    """Scale exponent p (scale s = 2**p) of the small kernels' pow2_scale.

    Restates tbf16/csrc/small_kernels.cu:12-18: e = clamp(E(amax), 1, 252),
    se = clamp(126 + t - (e - 127), 1, 254), s = 2**(se - 127). For a normal amax
    this puts amax * s in [2**(t-1), 2**t). Used by quantize_rows / quantize_cols
    (small_kernels.cu:61,172) and so by prepare_weight and the training ops.
    """
    e = np.clip(exp_field(amax), 1, 252)
    se = np.clip(253 + t - e, 1, 254)
    return (se - 127).astype(np.int32)


def pow2_exp_fused(amax, t: int) -> np.ndarray:
    """Fused GEMM row_scale variant, tbf16/csrc/gemm_sm75.cu:19-23: only the upper
    clamp on the biased scale exponent. Identical to pow2_exp for t >= 2 (the fused
    path always uses t = 15, tbf16/ops.py:26)."""
    e = np.clip(exp_field(amax), 1, 252)
    se = np.minimum(253 + t - e, 254)
    return (se - 127).astype(np.int32)


def pow2_exp_triton(amax, t: int) -> np.ndarray:
    """Triton fallback variant, tbf16/ops.py:39-45,57,66: 2**(126 - e) * 2**t with
    no clamp of the result. Returned as an exponent that may exceed 127 (the
    reference then holds inf). Kept only to document where the variants differ."""
    e = np.clip(exp_field(amax), 1, 252)
    return (126 - e + t).astype(np.int32)


def frexp_exp(v) -> np.ndarray:
    """torch.frexp exponent (v = m * 2**e, m in [0.5, 1); 0 for 0, inf, nan)."""
    m, e = np.frexp(np.asarray(v, dtype=np.float32))
    e = np.where(np.isfinite(np.asarray(v, dtype=np.float32)), e, 0)
    return e.astype(np.int32)


def target_exp(K: int) -> int:
    """tbf16/ops.py:29-32: rows scaled to amax in [2^(t-1), 2^t) keep |C| < K*4^t."""
    return min(0, (15 - math.ceil(math.log2(max(K, 1)))) // 2)


def dw_target_exp(M: int) -> int:
    """tbf16/autograd.py:85: |dW16| < M * 2^t must stay under fp16's max."""
    return min(0, 15 - math.ceil(math.log2(max(M, 1))))


def attn_do_target(D: int) -> int:
    """tbf16/autograd.py:176: t_do = 12 - ceil(log2 D)."""
    return 12 - math.ceil(math.log2(D))


L1_TARGET = 15            # tbf16/ops.py:130
FUSED_T = 15              # tbf16/ops.py:26
FUSED_MIN_M = 256         # tbf16/ops.py:23
SMALL_M = 2               # tbf16/ops.py:204


def ldexp1(p) -> np.ndarray:
    """float32 2**p (exact; 2**-127 is an fp32 subnormal and stays one)."""
    return np.ldexp(np.float32(1.0), np.asarray(p, dtype=np.int32)).astype(np.float32)


# ---------------------------------------------------------------------------
# Rounding helpers (bit-level, independent of torch's casts)
# ---------------------------------------------------------------------------

def bf16_bits_to_f32(bits) -> np.ndarray:
    b = np.asarray(bits, dtype=np.uint32) << 16
    return b.view(np.float32)


def f32_to_bf16_rne_bits(x) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even; NaN stays a quiet NaN."""
    u = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).view(np.uint32).astype(np.uint64)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


# ---------------------------------------------------------------------------
# a2 / a4 / a5 / a9: row and column quantisation
# ---------------------------------------------------------------------------

def row_amax(x: torch.Tensor, l1: bool) -> np.ndarray:
    """Per-row max |x| (exact) or L1 norm. The L1 norm is the exact sum rounded
    once to fp32; the reference sums in fp32 in thread order
    (small_kernels.cu:42-59), which can differ only when the sum lies within an
    fp32 ulp of a power of two."""
    xf = x.float()
    if l1:
        return xf.double().abs().sum(1).float().numpy()
    if xf.shape[1] == 0:
        return np.zeros(xf.shape[0], np.float32)
    # fmaxf in the reference's reduction skips NaN operands (small_kernels.cu:48)
    return torch.nan_to_num(xf.abs(), nan=0.0).amax(1).numpy()


def row_exps(x: torch.Tensor, t: int, l1: bool = False, fused: bool = False) -> np.ndarray:
    """Row scale exponents: quantize_rows (small_kernels.cu:35-74) or the fused
    GEMM's row_scale (gemm_sm75.cu:27-47)."""
    amax = row_amax(x, l1)
    return pow2_exp_fused(amax, t) if fused else pow2_exp(amax, t)


def quantize_rows(x: torch.Tensor, t: int = 0, l1: bool = False):
    """bf16 (R, K) -> (fp16 (R, K), fp32 s_inv (R,)).

    Restates quantize_rows (tbf16/ops.py:74-89 -> small_kernels.cu:35-74):
    y = fp16_rne(x * s) with s = 2**p from pow2_exp, s_inv = 1 / s.
    """
    p = row_exps(x, t, l1)
    s = torch.from_numpy(ldexp1(p))
    y = (x.float() * s[:, None]).half()
    return y, torch.from_numpy(ldexp1(-p))


def prepare_weight(w: torch.Tensor):
    """tbf16/ops.py:140-142: quantize_rows(w, target_exp(K))."""
    return quantize_rows(w.contiguous(), target_exp(w.shape[1]))


def quantize_cols(x: torch.Tensor, t: int = 0, row_mul: torch.Tensor | None = None):
    """bf16 (R, K) -> (fp16 (R, K), fp32 s_inv (K,)), one scale per column.

    Restates col_amax_kernel + col_convert_kernel (small_kernels.cu:136-184,
    318-340): amax[c] = max_r |x[r,c]| * |row_mul[r]|, y = fp16((x * row_mul) * s_c).
    R == 0 gives s_inv = 1 (small_kernels.cu:325).
    """
    R, K = x.shape
    if R == 0:
        return torch.empty(0, K, dtype=torch.float16), torch.ones(K)
    xf = x.float()
    rm = row_mul.float() if row_mul is not None else torch.ones(R)
    amax = (xf.abs() * rm.abs()[:, None]).amax(0).numpy()
    p = pow2_exp(amax, t)
    s = torch.from_numpy(ldexp1(p))
    y = ((xf * rm[:, None]) * s[None, :]).half()
    return y, torch.from_numpy(ldexp1(-p))


# ---------------------------------------------------------------------------
# a3 / a6 / a7 / a8: linear
# ---------------------------------------------------------------------------

def _epilogue(acc: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor, bias) -> torch.Tensor:
    """acc * sa[m] * sb[n] + bias[n] in fp32, one RNE rounding to bf16
    (gemm_sm75.cu:215-216, small_kernels.cu:94-99)."""
    y = acc.float() * sa.float()[:, None] * sb.float()[None, :]
    if bias is not None:
        y = y + bias.float()[None, :]
    return y.bfloat16()


def linear_fused(x: torch.Tensor, w16: torch.Tensor, ws: torch.Tensor, bias=None, t: int = FUSED_T,
                 l1: bool = False) -> torch.Tensor:
    """Fused GEMM (gemm_sm75.cu:78-226, 257-284): x rows scaled (row_scale),
    converted to fp16, fp32 accumulation, bf16 out from fp32 (single rounding)."""
    p = row_exps(x, t, l1, fused=not l1)
    x16 = (x.float() * torch.from_numpy(ldexp1(p))[:, None]).half()
    acc = x16.float() @ w16.float().t()
    return _epilogue(acc, torch.from_numpy(ldexp1(-p)), ws, bias)


def linear_cublas_path(x: torch.Tensor, w16: torch.Tensor, ws: torch.Tensor, bias=None) -> torch.Tensor:
    """The reference's 2 <= M < 256 regime (ops.py:163-178): L1 row scales at
    t = 15, an fp16 C (cuBLAS fp16 output) and then the bf16 epilogue. This double
    rounding is the reference's own error at small M."""
    x16, sx = quantize_rows(x, L1_TARGET, l1=True)
    c16 = (x16.float() @ w16.float().t()).half()
    return _epilogue(c16.float(), sx, ws, bias)


def linear_small_m(x: torch.Tensor, w16: torch.Tensor, ws: torch.Tensor, bias=None) -> torch.Tensor:
    """This build's 2 <= M < 256 path: the reference's L1 exponents (ops.py:163)
    with fp32 accumulation and a single bf16 rounding (no fp16 C)."""
    x16, sx = quantize_rows(x, L1_TARGET, l1=True)
    acc = x16.float() @ w16.float().t()
    return _epilogue(acc, sx, ws, bias)


def gemv(x: torch.Tensor, w16: torch.Tensor, ws: torch.Tensor, bias=None) -> torch.Tensor:
    """M = 1 (small_kernels.cu:107-132): fp32 dot of bf16 x with fp16 w, times
    ws, plus bias, one bf16 rounding. No activation scale."""
    acc = x.float().reshape(1, -1) @ w16.float().t()
    y = acc * ws.float()[None, :]
    if bias is not None:
        y = y + bias.float()[None, :]
    return y.bfloat16()


def scaled_linear(x: torch.Tensor, w16: torch.Tensor, ws: torch.Tensor, bias=None) -> torch.Tensor:
    """Dispatcher of tbf16/ops.py:153-164 as this build runs it: M < 2 -> GEMV,
    M >= 256 -> fused (max rows, t = 15), else L1 rows at t = 15; all with fp32
    accumulation and one bf16 rounding."""
    shape = x.shape
    x2 = x.reshape(-1, shape[-1])
    M = x2.shape[0]
    if M < SMALL_M:
        y = gemv(x2, w16, ws, bias) if M == 1 else torch.empty(0, w16.shape[0], dtype=torch.bfloat16)
    elif M >= FUSED_MIN_M:
        y = linear_fused(x2, w16, ws, bias)
    else:
        y = linear_small_m(x2, w16, ws, bias)
    return y.reshape(*shape[:-1], w16.shape[0])


def linear_ref64(x, w, bias=None) -> torch.Tensor:
    """fp64 reference of the same bf16 values (tests/test_ops.py:13)."""
    y = x.double() @ w.double().t()
    return y + bias.double() if bias is not None else y


# ---------------------------------------------------------------------------
# a10: training linear (autograd.py:58-90)
# ---------------------------------------------------------------------------

def linear_train_fwd(x2: torch.Tensor, w: torch.Tensor, bias=None, double_round: bool = False):
    """ScaledLinearFn.forward (autograd.py:60-68): x rows max-scaled at
    target_exp(K), w via prepare_weight, fp32 accumulation (double_round: the
    reference's fp16 GEMM output). Returns (y, x16, sx, w16, sw)."""
    K = w.shape[1]
    x16, sx = quantize_rows(x2, target_exp(K))
    w16, sw = prepare_weight(w)
    acc = x16.float() @ w16.float().t()
    if double_round:
        acc = acc.half().float()
    return _epilogue(acc, sx, sw, bias), x16, sx, w16, sw


def linear_train_bwd(dy2: torch.Tensor, x16: torch.Tensor, sx: torch.Tensor, w: torch.Tensor,
                     double_round: bool = False):
    """ScaledLinearFn.backward (autograd.py:71-90) with fp32 accumulation and one
    bf16 rounding per output; double_round=True also rounds the GEMM result to fp16
    first, as the reference's cuBLAS fp16 output does (its own error). Returns
    (dx, dw, db, exps) where exps holds every scale exponent the reference computes."""
    N, K = w.shape
    M = dy2.shape[0]
    rnd = (lambda c: c.half().float()) if double_round else (lambda c: c)
    dy16, sdy = quantize_rows(dy2, L1_TARGET, l1=True)
    w16c, swc = quantize_cols(w.contiguous(), target_exp(N))
    dx = _epilogue(rnd(dy16.float() @ w16c.float()), sdy, swc, None)
    t = dw_target_exp(M)
    dy16c, sdyc = quantize_cols(dy2, t, sx)
    dw = _epilogue(rnd(dy16c.float().t() @ x16.float()), sdyc, torch.ones(K), None)
    db = dy2.float().sum(0).to(dy2.dtype)
    exps = {"sdy": sdy, "swc": swc, "sdyc": sdyc}
    return dx, dw, db, exps


# ---------------------------------------------------------------------------
# a11 - a15: attention
# ---------------------------------------------------------------------------

def head_amax(x: torch.Tensor) -> torch.Tensor:
    """small_kernels.cu:222-243: max |x[b, h]| over (S, D), fp32 (B, H)."""
    if x.shape[2] == 0 or x.shape[3] == 0:
        return torch.zeros(x.shape[0], x.shape[1])
    return x.float().abs().amax(dim=(-2, -1))


def head_exp(x: torch.Tensor) -> torch.Tensor:
    """tbf16/attention.py:24-27: frexp exponent of each head's amax, int32."""
    return torch.frexp(head_amax(x))[1].to(torch.int32)


def attn_exponents(q, k, v, v_exp: int):
    """prepare_qkv exponents (attention.py:38-48): a (scalar) and ev (B, Hkv)."""
    eq = int(head_exp(q).max())
    ek = int(head_exp(k).max())
    a = (ek - eq) // 2
    a = max(min(a, 14 - eq), ek - 14)
    ev = head_exp(v) - v_exp
    return a, ev


def head_scale(x: torch.Tensor, e: torch.Tensor, dtype) -> torch.Tensor:
    """attention.py:30-35: x * 2**e[b, h] cast to dtype (contiguous)."""
    e = e.to(torch.int32).expand(x.shape[0], x.shape[1])
    s = torch.ldexp(torch.ones(e.shape), e.float())
    return (x.float() * s[..., None, None]).to(dtype).contiguous()


def expand_heads(e: torch.Tensor, n_heads: int) -> torch.Tensor:
    """attention.py:51-53."""
    return e if e.shape[1] == n_heads else e.repeat_interleave(n_heads // e.shape[1], dim=1)


def prepare_qkv(q, k, v, v_exp: int = 0):
    """attention.py:38-48: scaled fp16 copies and the exponents."""
    a, ev = attn_exponents(q, k, v, v_exp)
    at = torch.tensor([[a]], dtype=torch.int32)
    q16 = head_scale(q, at, torch.float16)
    k16 = head_scale(k, -at, torch.float16)
    v16 = head_scale(v, -ev, torch.float16)
    return q16, k16, v16, a, ev


def causal_mask(Sq: int, Sk: int) -> torch.Tensor:
    """is_causal: query i sees keys j <= i (top-left aligned, as torch SDPA)."""
    return torch.ones(Sq, Sk, dtype=torch.bool).tril(0)


def sdpa_ref64(q, k, v, causal=False, scale=None, mask=None, rows=None):
    """fp64 softmax(q k^T * scale + mask) v of the same bf16 values
    (tests/test_attention.py:7-13). `rows` restricts the query rows (each row
    depends only on its own q and all of k, v). GQA by repeating kv heads."""
    qd, kd, vd = q.double(), k.double(), v.double()
    H, Hkv = q.shape[1], k.shape[1]
    if Hkv != H:
        kd = kd.repeat_interleave(H // Hkv, 1)
        vd = vd.repeat_interleave(H // Hkv, 1)
    D = q.shape[-1]
    sc = (1.0 / math.sqrt(D)) if scale is None else scale
    Sq, Sk = q.shape[2], k.shape[2]
    idx = torch.arange(Sq) if rows is None else torch.as_tensor(rows)
    s = (qd[:, :, idx] @ kd.transpose(-1, -2)) * sc
    if causal:
        allowed = causal_mask(Sq, Sk)[idx]
        s = s.masked_fill(~allowed, float("-inf"))
    if mask is not None:
        m = mask[..., idx, :] if mask.shape[-2] == Sq and Sq > 1 else mask
        s = s.masked_fill(~m, float("-inf")) if m.dtype == torch.bool else s + m.double()
    return torch.softmax(s, -1) @ vd


def sdpa_fp16_emulated(q, k, v, causal=False, scale=None, v_exp=13, rows=None):
    """This build's attention arithmetic on the CPU: fp16 copies scaled by
    2^a, 2^-a, 2^-ev (attention.py:38-48), logits and softmax in fp32, P
    rounded to fp16 for P.V, fp32 accumulation, out = bf16(O / l * 2^ev) with one
    rounding. The reference itself rounds O to fp16 first (attention.py:63-65)."""
    q16, k16, v16, a, ev = prepare_qkv(q, k, v, v_exp)
    H, Hkv = q.shape[1], k.shape[1]
    k16e = k16.repeat_interleave(H // Hkv, 1) if Hkv != H else k16
    v16e = v16.repeat_interleave(H // Hkv, 1) if Hkv != H else v16
    D = q.shape[-1]
    sc = (1.0 / math.sqrt(D)) if scale is None else scale
    Sq, Sk = q.shape[2], k.shape[2]
    idx = torch.arange(Sq) if rows is None else torch.as_tensor(rows)
    s = (q16[:, :, idx].float() @ k16e.float().transpose(-1, -2)) * sc
    if causal:
        s = s.masked_fill(~causal_mask(Sq, Sk)[idx], float("-inf"))
    m = s.amax(-1, keepdim=True)
    p = torch.exp(s - m)
    l = p.sum(-1, keepdim=True)
    o = (p.half().float() @ v16e.float()) / l
    evq = expand_heads(ev, H).float()
    return (o * torch.ldexp(torch.ones_like(evq), evq)[..., None, None]).bfloat16(), a, ev


def sdpa_reference_arith(q, k, v, causal=False, scale=None, v_exp=13, rows=None):
    """The reference's own inference arithmetic (attention.py:56-65), restated so
    tests can hold this build to "no worse than the reference's error": prepare_qkv's
    fp16 copies, then what torch's fp16 memory-efficient kernel computes (logits,
    row max and softmax sums in fp32, P rounded to fp16 for the P.V product with fp32
    accumulation, O / l rounded to fp16 as its fp16 output), then head_scale of that
    fp16 output by 2^ev into bf16: two roundings of the output. One softmax over the
    whole row replaces the kernel's per-tile online rescaling (the same values up to
    fp32 rounding). Works on any device; per (b, h) to bound memory."""
    q16, k16, v16, a, ev = prepare_qkv(q.cpu(), k.cpu(), v.cpu(), v_exp)
    dev = q.device
    q16, k16, v16 = q16.to(dev), k16.to(dev), v16.to(dev)
    B, H, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    sc = (1.0 / math.sqrt(D)) if scale is None else scale
    idx = torch.arange(Sq, device=dev) if rows is None else torch.as_tensor(rows, device=dev)
    kj = torch.arange(Sk, device=dev)
    evq = expand_heads(ev, H)
    out = torch.empty(B, H, len(idx), D, dtype=torch.bfloat16, device=dev)
    for b in range(B):
        for h in range(H):
            hk = h // (H // Hkv)
            s = (q16[b, h, idx].float() @ k16[b, hk].float().t()) * sc
            if causal:
                s = s.masked_fill(kj[None, :] > idx[:, None], float("-inf"))
            m = s.amax(-1, keepdim=True)
            p = torch.exp(s - m)
            l = p.sum(-1, keepdim=True)
            o16 = ((p.half().float() @ v16[b, hk].float()) / l).half()
            out[b, h] = (o16.float() * math.ldexp(1.0, int(evq[b, h]))).bfloat16()
    return out


def sdpa_bwd_reference_arith(q, k, v, dout, causal=False, scale=None):
    """The reference's training attention arithmetic (autograd.py:149-193) restated
    on any device: prepare_qkv(v_exp=0) copies; the fp16 forward (as
    sdpa_reference_arith, O / l rounded to fp16 = out16, its lse kept in fp32); e
    and the first G from attn_bwd_exponents; then per attempt dO16 = fp16(dout
    2^(ev_q + G)) and what the memory-efficient fp16 backward computes: P = exp(s -
    lse) in fp32, rounded to fp16 for dV = P^T dO16; dP = dO16 V16^T and delta =
    rowsum(dO16 o out16) in fp32; dS = P (dP - delta) rounded to fp16 for dQ =
    scale dS K16 and dK = scale dS^T Q16; each gradient accumulated in fp32 and
    rounded to fp16 per query head (dq16, dk16, dv16). If any of those is not finite
    the attempt is redone at t_do - 8 (at most 6 attempts, autograd.py:177-189) --
    the check sees every query head's fp16 gradient before a GQA group is summed in
    fp32 (autograd.py:141-146, 180-186). The accepted attempt is head_scale'd by
    2^(a-G), 2^(-a-G), 2^(-ev-G) into bf16. Returns (out bf16, dq, dk, dv bf16,
    (a, ev, e, G))."""
    dev = q.device
    B, H, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    q16, k16, v16, a, ev = prepare_qkv(q.cpu(), k.cpu(), v.cpu(), 0)
    q16, k16, v16 = q16.to(dev), k16.to(dev), v16.to(dev)
    evq = expand_heads(ev, H)
    e, t_do, _ = attn_bwd_exponents(dout.cpu(), evq, D)
    sc = (1.0 / math.sqrt(D)) if scale is None else scale
    qi = torch.arange(Sq, device=dev)
    kj = torch.arange(Sk, device=dev)
    out = torch.empty(B, H, Sq, D, dtype=torch.bfloat16, device=dev)
    # the forward (out16, lse) per head, shared by every attempt
    fwd = {}
    for b in range(B):
        for h in range(H):
            hk = h // (H // Hkv)
            Q, K, V = q16[b, h].float(), k16[b, hk].float(), v16[b, hk].float()
            s = (Q @ K.t()) * sc
            if causal:
                s = s.masked_fill(kj[None, :] > qi[:, None], float("-inf"))
            m = s.amax(-1, keepdim=True)
            p = torch.exp(s - m)
            l = p.sum(-1, keepdim=True)
            o16 = ((p.half().float() @ V) / l).half()
            out[b, h] = (o16.float() * math.ldexp(1.0, int(evq[b, h]))).bfloat16()
            fwd[b, h] = (s, o16, m + torch.log(l))

    def attempt(G):
        dq16 = torch.empty(B, H, Sq, D, dtype=torch.float16, device=dev)
        dk32 = torch.zeros(B, Hkv, Sk, D, dtype=torch.float32, device=dev)
        dv32 = torch.zeros_like(dk32)
        finite = True
        for b in range(B):
            for h in range(H):
                hk = h // (H // Hkv)
                Q, K, V = q16[b, h].float(), k16[b, hk].float(), v16[b, hk].float()
                s, o16, lse = fwd[b, h]
                do16 = (dout[b, h].float() * math.ldexp(1.0, int(evq[b, h]) + G)).half().float()
                P = torch.exp(s - lse)
                dv16 = (P.half().float().t() @ do16).half()
                dP = do16 @ V.t()
                delta = (do16 * o16.float()).sum(-1, keepdim=True)
                dS = (P * (dP - delta)).half().float()
                dq16[b, h] = ((dS @ K) * sc).half()
                dk16 = ((dS.t() @ Q) * sc).half()
                finite &= bool(torch.isfinite(dq16[b, h]).all() and torch.isfinite(dk16).all()
                               and torch.isfinite(dv16).all())
                dk32[b, hk] += dk16.float()
                dv32[b, hk] += dv16.float()
        return dq16, dk32, dv32, finite

    for _ in range(6):
        G = t_do - e
        dq16, dk32, dv32, finite = attempt(G)
        if finite:
            break
        t_do -= 8
    else:
        raise FloatingPointError("tbf16 attention backward overflowed fp16 even after rescaling")
    dq = (dq16.float() * math.ldexp(1.0, a - G)).bfloat16()
    # (with Hkv == H each sum holds one fp16 value, which head_scale scales directly)
    sv = torch.tensor([[math.ldexp(1.0, -int(ev[b, h]) - G) for h in range(Hkv)] for b in range(B)],
                      dtype=torch.float32, device=dev)
    dk = (dk32 * math.ldexp(1.0, -a - G)).bfloat16()
    dv = (dv32 * sv[:, :, None, None]).bfloat16()
    return out, dq, dk, dv, (a, ev, e, G)


def attn_bwd_exponents(dout: torch.Tensor, ev_q: torch.Tensor, D: int):
    """autograd.py:175-176: e = max(head_exp(dO) + ev_q), t_do = 12 - ceil(log2 D),
    G = t_do - e (first attempt)."""
    e = int((head_exp(dout) + ev_q).max())
    t_do = attn_do_target(D)
    return e, t_do, t_do - e


def attn_bwd_retry(e: int, t_do: int, overflowed, attempts: int = 6):
    """autograd.py:177-189: try G = t_do - e; on overflow t_do -= 8; after
    `attempts` failures raise FloatingPointError. `overflowed(G)` says whether the
    backward at that G overflowed fp16. Returns the G that was accepted."""
    for _ in range(attempts):
        G = t_do - e
        if not overflowed(G):
            return G
        t_do -= 8
    raise FloatingPointError("tbf16 attention backward overflowed fp16 even after rescaling")


def sdpa_grads_ref64(q, k, v, dout, causal=False, scale=None, mask=None):
    """fp64 autograd of softmax attention on the same bf16 values
    (tests/test_autograd.py:15-19, 34-42). Returns (o, dq, dk, dv)."""
    qd, kd, vd = (t.detach().double().requires_grad_() for t in (q, k, v))
    o = sdpa_ref64(qd, kd, vd, causal, scale, mask)
    o.backward(dout.double())
    return o.detach(), qd.grad, kd.grad, vd.grad


def rel_err(y, ref) -> float:
    """Relative Frobenius error ||y - ref|| / ||ref|| (tests/test_accuracy.py:6-7)."""
    y, ref = y.double(), ref.double()
    return float((y - ref).norm() / ref.norm())


# ---------------------------------------------------------------------------
# Attention dropout keep mask: this build's definition (the kernels' device
# helpers drop_row / drop_pair / drop_keep); the reference passes dropout_p to
# torch's kernel, whose Philox-based mask is not comparable bit for bit.
# ---------------------------------------------------------------------------

_U32 = np.uint32


def fmix32(h) -> np.ndarray:
    """MurmurHash3's 32-bit finalizer (A. Appleby, public domain), elementwise on
    uint32 with wrap-around multiplication."""
    h = np.array(h, dtype=np.uint64) & 0xFFFFFFFF
    h ^= h >> 16
    h = (h * 0x85EBCA6B) & 0xFFFFFFFF
    h ^= h >> 13
    h = (h * 0xC2B2AE35) & 0xFFFFFFFF
    h ^= h >> 16
    return h.astype(_U32)


def dropout_params(p: float):
    """(thr16, scale) as the C ABI derives them from a float32 dropout_p:
    thr16 = min(65535, floor(p * 65536 + 0.5)), at least 1 for p > 0;
    scale = fp32(1 / (1 - p))."""
    p32 = np.float32(p)
    if p32 <= 0:
        return 0, np.float32(1.0)
    thr = int(min(65535.0, float(p32) * 65536.0 + 0.5))
    thr = max(thr, 1)
    return thr, np.float32(1.0) / (np.float32(1.0) - p32)


def dropout_keep(seed: int, bh: int, Sq: int, rows, cols, p: float) -> np.ndarray:
    """Keep mask (len(rows), len(cols)) of query head bh = b * H + h:
    row = fmix32((bh * Sq + q) ^ seed_lo), u = fmix32(row + (k >> 1) * 0x9E3779B9 +
    seed_hi), key k kept iff its 16-bit half of u (low half for even k) >= thr16."""
    thr, _ = dropout_params(p)
    lo, hi = seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF
    q = np.asarray(rows, dtype=np.uint64)
    k = np.asarray(cols, dtype=np.uint64)
    row = fmix32(((bh * Sq + q) & 0xFFFFFFFF) ^ lo).astype(np.uint64)
    u = fmix32((row[:, None] + ((k[None, :] >> 1) * 0x9E3779B9) + hi) & 0xFFFFFFFF).astype(np.uint64)
    half = np.where((k[None, :] & 1) == 1, u >> 16, u & 0xFFFF)
    return half >= thr


def dropout_z(seed: int, B: int, H: int, Sq: int, Sk: int, p: float) -> torch.Tensor:
    """Z = keep / (1 - p) as float64 (B, H, Sq, Sk): the dropped attention weights are
    softmax(S) * Z."""
    _, scale = dropout_params(p)
    z = np.empty((B, H, Sq, Sk), dtype=np.float64)
    for b in range(B):
        for h in range(H):
            z[b, h] = dropout_keep(seed, b * H + h, Sq, np.arange(Sq), np.arange(Sk), p) * float(scale)
    return torch.from_numpy(z)


# ---------------------------------------------------------------------------
# Scaled convolutions (tbf16/conv.py): per-sample input exponents, the scaled
# fp16 input, the fp16 convolution (emulated) and the bf16 epilogue.
# ---------------------------------------------------------------------------

def conv_sample_exps(x: torch.Tensor, t: int) -> np.ndarray:
    """tbf16/conv.py:28-31,49-50: e[b] = frexp(max |x[b]|) - t, where the max-norm
    propagates NaN and an amax that is not > 0 (zero or NaN) is taken as 1; an
    infinite amax has frexp exponent 0."""
    B = x.shape[0]
    if B == 0:
        return np.zeros((0,), dtype=np.int32)
    amax = x.detach().float().reshape(B, -1).abs().amax(dim=1).numpy()
    amax = np.where(amax > 0, amax, np.float32(1.0))
    return (frexp_exp(amax) - t).astype(np.int32)


def conv_scale_input(x: torch.Tensor, e) -> torch.Tensor:
    """tbf16/conv.py:51-54: fp16(x * ldexp(1, -e[b])) with the scale an fp32 power of
    two (inf for -e >= 128) and one RNE rounding of the fp32 product."""
    e = np.asarray(e, dtype=np.int32)
    s = torch.from_numpy(ldexp1(-e)).view((-1,) + (1,) * (x.dim() - 1))
    return (x.float() * s).half()


def conv_epilogue(y16: torch.Tensor, e, ws: torch.Tensor, bias=None) -> torch.Tensor:
    """tbf16/conv.py:56-60: bf16(y16 * (2^e[b] * ws[o]) + bias[o]): the scale is the fp32
    product of two powers of two, y16 * scale and the bias add are fp32 operations,
    the result is rounded once more to bf16."""
    B, O = y16.shape[:2]
    view = (B, O) + (1,) * (y16.dim() - 2)
    scale = (torch.from_numpy(ldexp1(np.asarray(e, dtype=np.int32)))[:, None] * ws.float()[None, :]).view(view)
    r = y16.float() * scale
    if bias is not None:
        r = r + bias.float().view((1, O) + (1,) * (y16.dim() - 2))
    return r.bfloat16()


_CONV_FNS = {1: F.conv1d, 2: F.conv2d, 3: F.conv3d}


def conv_weight(w: torch.Tensor):
    """tbf16/conv.py:89-97: the weight as (fp16 of its shape, fp32 (O,) inverse scales),
    one max scale per output channel at t = target_exp(C_in / groups * prod(kernel))."""
    O = w.shape[0]
    w16, ws = prepare_weight(w.reshape(O, -1))
    return w16.reshape(w.shape), ws


def conv_forward(x: torch.Tensor, w16: torch.Tensor, ws: torch.Tensor, bias=None, stride=1, padding=0,
                 dilation=1, groups=1) -> torch.Tensor:
    """tbf16/conv.py:39-60 (zero padding) on the CPU: exponents, scaled input, an fp16
    convolution emulated as the exact (fp64) sum rounded to fp16 -- the library
    accumulates in fp32, so this is its error up to the fp32 accumulation -- and
    the epilogue. The input must be batched."""
    nd = x.dim() - 2
    t = target_exp(w16[0].numel())
    e = conv_sample_exps(x, t)
    x16 = conv_scale_input(x, e)
    y = _CONV_FNS[nd](x16.double(), w16.double(), None, stride, padding, dilation, groups)
    return conv_epilogue(y.half(), e, ws, bias)


def conv_ref64(x: torch.Tensor, w: torch.Tensor, bias=None, stride=1, padding=0, dilation=1, groups=1,
               padding_mode: str = "zeros", reversed_padding=None) -> torch.Tensor:
    """The reference's accuracy oracle (tests/test_conv.py:15-21): the fp64 convolution
    of the same bf16 input with the dequantized weight."""
    nd = x.dim() - 2
    b = None if bias is None else bias.double()
    if padding_mode != "zeros":
        xp = F.pad(x.double(), reversed_padding, mode=padding_mode)
        return _CONV_FNS[nd](xp, w.double(), b, stride, 0, dilation, groups)
    return _CONV_FNS[nd](x.double(), w.double(), b, stride, padding, dilation, groups)
