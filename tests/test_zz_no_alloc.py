"""ar_linear_bwd_dw_bf16_noalloc (scratch in a fixed device array, no
workspace, no allocation) against ar_linear_bwd_dw_bf16 (scratch from the
bound workspace): the same kernels and split counts, so the accumulated dW
must be bit-identical.  Calls run back to back on a stream with no workspace
bound, the second and third on smaller inputs than the first (the array keeps
the previous call's contents)."""
import ctypes as ct

import numpy as np
import pytest

import gpu_util as gu

pytestmark = pytest.mark.gpu

LIMIT = 64 << 20  # bytes of the fixed scratch array (include/ar_ops.h)


def _ptr(t):
    return ct.c_void_p(t.data_ptr())


def _inputs(seed, M, N, K):
    r = gu.rng(seed)
    dY = gu.randn(r, M, N)
    X = gu.randn(r, M, K)
    dW0 = gu.randn(r, N, K, scale=0.1)
    return dY, X, dW0


def test_noalloc_matches_workspace_entry():
    import torch
    from autoresearch_amd import _lib
    lib = _lib.load()
    side = torch.cuda.Stream()  # default priority; no workspace is bound to it
    cases = [
        (65536, 512, 512),   # benchmark q / k / v dW shape: 64 split-K partials, the whole array
        (4096, 256, 384),    # smaller: fewer partials over the previous call's contents
        (1001, 70, 43),      # off the 8-multiple grid: zero-padded operand copies in the array
    ]
    for i, (M, N, K) in enumerate(cases):
        dY, X, dW0 = _inputs(100 + i, M, N, K)
        dYd, Xd = gu.dev(dY), gu.dev(X)
        ref = gu.dev(dW0)
        out = gu.dev(dW0)
        print(f"[noalloc] case {i}: M={M} N={N} K={K}", flush=True)
        # existing entry: workspace bound to the default stream by conftest
        _lib.check(lib.ar_linear_bwd_dw_bf16(None, _ptr(ref), _ptr(dYd), _ptr(Xd), M, N, K), "linear_bwd_dw_bf16")
        torch.cuda.synchronize()
        call = lambda o: _lib.check(lib.ar_linear_bwd_dw_bf16_noalloc(  # noqa: E731
            ct.c_void_p(side.cuda_stream), _ptr(o), _ptr(dYd), _ptr(Xd), M, N, K), "linear_bwd_dw_bf16_noalloc")
        call(out)
        side.synchronize()
        # the same call again: the device's free memory does not move (the
        # first call of a shape may still make the runtime load code or
        # grow its own kernel scratch, so it is not the one measured)
        again = gu.dev(dW0)
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        call(again)
        side.synchronize()
        assert torch.cuda.mem_get_info()[0] == free0
        a, b = gu.host(out), gu.host(ref)
        assert np.all(np.isfinite(a))
        np.testing.assert_array_equal(a, b)
        np.testing.assert_array_equal(gu.host(again), b)
        # and it is the product (bf16 operands, fp32 accumulation): dW0 + dY^T X
        want = dW0.astype(np.float64) + dY.astype(np.float64).T @ X.astype(np.float64)
        err = np.linalg.norm(a - want) / np.linalg.norm(want)
        assert err <= 2e-2, err


def test_noalloc_rejects_shapes_beyond_the_array():
    import torch
    from autoresearch_amd import _lib
    lib = _lib.load()
    # M off the 8-multiple grid: the padded copy of dY alone is > 64 MiB
    M, N, K = 65537, 512, 512
    dY = torch.zeros(M, N, device="cuda")
    X = torch.zeros(M, K, device="cuda")
    dW = torch.full((N, K), 3.0, device="cuda")
    st = lib.ar_linear_bwd_dw_bf16_noalloc(None, _ptr(dW), _ptr(dY), _ptr(X), M, N, K)
    assert st == -1
    msg = lib.ar_last_error().decode()
    assert "scratch" in msg and str(LIMIT) in msg, msg
    torch.cuda.synchronize()
    assert torch.all(dW == 3.0)  # nothing ran
