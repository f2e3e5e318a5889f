"""tbf16_linear_noalloc (its workspace in the library's static device scratch array)
against tbf16_linear (workspace from the caller): the same output bit for bit on two
calls in a row, the second one smaller, through the C ABI; and calls beyond the
scratch limit are rejected before any launch."""
import ctypes

import pytest
import torch

from tbf16 import _ext, ops

pytestmark = pytest.mark.gpu


def _inputs(dev, M, K, N, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(M, K, generator=g) * torch.ldexp(torch.ones(M, 1), torch.randint(-20, 21, (M, 1), generator=g)
                                                      .float())).bfloat16().to(dev)
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16().to(dev)
    b = torch.randn(N, generator=g).bfloat16().to(dev)
    w16, ws = ops.prepare_weight(w)
    return x, w16, ws, b


def _with_workspace(x, w16, ws, b, t, l1):
    M, K = x.shape
    N = w16.shape[0]
    y = torch.empty(M, N, dtype=torch.bfloat16, device=x.device)
    work = torch.empty(int(_ext.lib().tbf16_linear_ws_bytes(M, K, N, -1)), dtype=torch.uint8, device=x.device)
    _ext.call("tbf16_linear", x.data_ptr(), M, K, K, w16.data_ptr(), N, K, ws.data_ptr(), b.data_ptr(), y.data_ptr(),
              N, t, l1, -1, work.data_ptr(), _ext.stream())
    return y


def _no_alloc(x, w16, ws, b, t, l1):
    M, K = x.shape
    N = w16.shape[0]
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=x.device)
    _ext.call("tbf16_linear_noalloc", x.data_ptr(), M, K, K, w16.data_ptr(), N, K, ws.data_ptr(), b.data_ptr(),
              y.data_ptr(), N, t, l1, -1, _ext.stream())
    return y


def test_noalloc_matches_workspace_entry_point(dev):
    # first call: 4096 rows (the fused max-scaled path); then, smaller, 200 rows with L1
    # row scales (256-row tiles) and 64 rows against N = 10240 (the decode kernel, its
    # fp16 copy of x in the scratch array), each overwriting the previous call's
    for (M, K, N, t, l1, seed) in ((4096, 2048, 1024, 15, 0, 1), (200, 2560, 768, 15, 1, 2),
                                   (64, 2560, 10240, 15, 1, 3)):
        x, w16, ws, b = _inputs(dev, M, K, N, seed)
        want = _with_workspace(x, w16, ws, b, t, l1)
        got = _no_alloc(x, w16, ws, b, t, l1)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (M, K, N)


def test_noalloc_rejects_rows_beyond_limit(dev):
    L = _ext.lib()
    limit = 1 << 20
    rc = L.tbf16_linear_noalloc(16, limit + 1, 8, 8, 16, 8, 8, 16, None, 16, 8, 15, 0, -1, None)
    assert rc == -1 and "scratch limit" in L.tbf16_last_error().decode()
    # a decode-sized call whose fp16 copy of x would not fit the array
    K = 32768
    assert L.tbf16_linear_ws_bytes(255, K, 10240, 18) > (12 << 20)
    rc = L.tbf16_linear_noalloc(16, 255, K, K, 16, 10240, K, 16, None, 16, 10240, 15, 1, 18, None)
    assert rc == -1 and "scratch limit" in L.tbf16_last_error().decode()
