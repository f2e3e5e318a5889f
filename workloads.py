"""Synthetic inputs for the five benchmark configurations.

Every tensor comes from a CPU `torch.Generator().manual_seed(seed)` and is cast
to bf16 (round to nearest even) on the CPU, so the same values can be moved to
any device. Shapes and distributions follow the configs this build is measured
on (scaled GEMM, small-M decode linear, scaled attention, training step).
"""
from __future__ import annotations

import torch


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def cfg1_cpu_linear(seed: int = 0):
    """Config 1: X bf16 (256, 4096) ~ N(0,1) with 13 rows (5 %) multiplied by 2^17
    (beyond fp16's range), W bf16 (4096, 4096) ~ N(0, 0.02), no bias."""
    g = _gen(seed)
    x = torch.randn(256, 4096, generator=g)
    rows = torch.randperm(256, generator=g)[:13]
    x[rows] *= 2.0 ** 17
    w = torch.randn(4096, 4096, generator=g) * 0.02
    return x.bfloat16(), w.bfloat16(), None


def cfg2_square_gemm(seed: int = 0, n: int = 4096):
    """Config 2: M = N = K = 4096; each row of X and of W is N(0,1) * 2^e with
    e uniform integer in [-20, 20], drawn independently for X and W."""
    g = _gen(seed)
    x = torch.randn(n, n, generator=g)
    ex = torch.randint(-20, 21, (n,), generator=g)
    w = torch.randn(n, n, generator=g)
    ew = torch.randint(-20, 21, (n,), generator=g)
    x = x * torch.ldexp(torch.ones(n), ex.float())[:, None]
    w = w * torch.ldexp(torch.ones(n), ew.float())[:, None]
    return x.bfloat16(), w.bfloat16(), None


CFG3_MS = (1, 16, 64, 255)


def cfg3_small_m(seed: int = 0, K: int = 2560, N: int = 10240, ms=CFG3_MS):
    """Config 3: W bf16 (10240, 2560) ~ N(0, 0.02) (MLP up-projection) and, per M,
    X bf16 (M, 2560) ~ N(0,1) with rows scaled by 2^e, e uniform integer in [0, 16].
    Returns (w, {M: x})."""
    g = _gen(seed)
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    xs = {}
    for M in ms:
        x = torch.randn(M, K, generator=g)
        e = torch.randint(0, 17, (M,), generator=g)
        xs[M] = (x * torch.ldexp(torch.ones(M), e.float())[:, None]).bfloat16()
    return w, xs


def cfg4_attention(S: int, seed: int = 0, B: int = 1, H: int = 16, D: int = 128):
    """Config 4: causal attention, q and k = N(0,1) * 2^u with u ~ U[0, 10] per
    head (independently for q and k), v = N(0,1) * 2^w with w ~ U[-4, 12] per head."""
    g = _gen(seed)

    def head_scaled(lo, hi):
        t = torch.randn(B, H, S, D, generator=g)
        u = lo + (hi - lo) * torch.rand(B, H, generator=g)
        return (t * torch.exp2(u)[..., None, None]).bfloat16()

    q = head_scaled(0.0, 10.0)
    k = head_scaled(0.0, 10.0)
    v = head_scaled(-4.0, 12.0)
    return q, k, v


def cfg5_train_linear(seed: int = 0, M: int = 8192, K: int = 2048, N: int = 6144):
    """Config 5, linear part: X rows N(0,1) * 2^e (e uniform integer in [0, 16]),
    W = N(0,1) * K^-0.5, dY = N(0,1) * 1e-3."""
    g = _gen(seed)
    x = torch.randn(M, K, generator=g)
    e = torch.randint(0, 17, (M,), generator=g)
    x = x * torch.ldexp(torch.ones(M), e.float())[:, None]
    w = torch.randn(N, K, generator=g) * K ** -0.5
    dy = torch.randn(M, N, generator=g) * 1e-3
    return x.bfloat16(), w.bfloat16(), dy.bfloat16()


def cfg5_train_attention(seed: int = 0, B: int = 2, H: int = 16, S: int = 4096, D: int = 128):
    """Config 5, attention part: q, k, v ~ N(0,1), dO ~ N(0, 2^-20), causal."""
    g = _gen(seed)
    q, k, v = (torch.randn(B, H, S, D, generator=g).bfloat16() for _ in range(3))
    do = (torch.randn(B, H, S, D, generator=g) * 2.0 ** -20).bfloat16()
    return q, k, v, do
