"""GEMM, flash attention and Muon parity on the GPU (through the C ABI).

Small shapes compare against the CPU oracle; the BASELINE config-2 /
config-3 shapes compare against a torch fp32 reference on the GPU (the oracle
would take minutes there), with the tolerance stated per test."""
import numpy as np
import pytest

from conftest import TOL_BF16, TOL_FP32, rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch  # noqa: F401
    from autoresearch_amd import ops
    from oracle import oracle as orc
    import gpu_util as gu
    return ops, orc, gu


GEMM_SHAPES = [(256, 256, 256), (384, 136, 520), (128, 512, 2048), (2048, 512, 128), (64, 8, 64)]


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
@pytest.mark.parametrize("bf16", [False, True])
def test_gemm_layouts_vs_oracle(env, M, N, K, bf16):
    ops, orc, gu = env
    r = gu.rng(M + N + K)
    tol = TOL_BF16 if bf16 else TOL_FP32
    X = gu.randn(r, M, K)
    W = gu.randn(r, N, K, scale=0.05)
    ref = np.zeros((M, N), np.float32)
    orc.call("linear_fwd", ref, X, W, M, N, K)
    out = gu.empty(M, N)
    ops.linear_fwd(out, gu.dev(X), gu.dev(W), M, N, K, bf16=bf16)
    assert rel_err(gu.host(out), ref) <= tol
    dY = gu.randn(r, M, N)
    ref = np.zeros((M, K), np.float32)
    orc.call("linear_bwd_dx", ref, dY, W, M, N, K)
    dx = gu.empty(M, K)
    ops.linear_bwd_dx(dx, gu.dev(dY), gu.dev(W), M, N, K, bf16=bf16)
    assert rel_err(gu.host(dx), ref) <= tol
    dw0 = gu.randn(r, N, K)
    ref = dw0.copy()
    orc.call("linear_bwd_dw", ref, dY, X, M, N, K)  # accumulates
    dw = gu.dev(dw0)
    ops.linear_bwd_dw(dw, gu.dev(dY), gu.dev(X), M, N, K, bf16=bf16)
    assert rel_err(gu.host(dw), ref) <= tol


@pytest.mark.parametrize("M,N,K", [(13, 24, 40), (1, 1, 1), (37, 129, 3), (300, 77, 515)])
@pytest.mark.parametrize("bf16", [False, True])
def test_gemm_any_shape_vs_oracle(env, M, N, K, bf16):
    """Any M, N, K (and operands only 4-byte aligned): the tail path pads into
    the workspace, as the reference's tiles bound-check every element
    (ops.mojo:150-168); dX in place (model.mojo:906) included."""
    ops, orc, gu = env
    import torch
    r = gu.rng(M * 7 + N * 3 + K)
    tol = TOL_BF16 if bf16 else TOL_FP32
    X, W, dY = gu.randn(r, M, K), gu.randn(r, N, K, scale=0.05), gu.randn(r, M, N)

    def unaligned(a):
        # a view starting 4 bytes into a fresh buffer: not 16-byte aligned
        buf = torch.empty(a.size + 1, dtype=torch.float32, device="cuda")
        v = buf[1:]
        v.copy_(torch.from_numpy(a.ravel()).cuda())
        return v

    ref = np.zeros((M, N), np.float32)
    orc.call("linear_fwd", ref, X, W, M, N, K)
    out = unaligned(np.full((M, N), np.nan, np.float32))
    ops.linear_fwd(out, unaligned(X), gu.dev(W), M, N, K, bf16=bf16)
    assert rel_err(gu.host(out).reshape(M, N), ref) <= tol
    ref = np.zeros((M, K), np.float32)
    orc.call("linear_bwd_dx", ref, dY, W, M, N, K)
    dx = gu.empty(M, K)
    ops.linear_bwd_dx(dx, gu.dev(dY), unaligned(W), M, N, K, bf16=bf16)
    assert rel_err(gu.host(dx), ref) <= tol
    if N == K:
        buf = gu.dev(dY)
        ops.linear_bwd_dx(buf, buf, gu.dev(W), M, N, K, bf16=bf16)
        assert rel_err(gu.host(buf), ref) <= tol
    dw0 = gu.randn(r, N, K)
    ref = dw0.copy()
    orc.call("linear_bwd_dw", ref, dY, X, M, N, K)
    dw = unaligned(dw0)
    ops.linear_bwd_dw(dw, gu.dev(dY), gu.dev(X), M, N, K, bf16=bf16)
    assert rel_err(gu.host(dw).reshape(N, K), ref) <= tol


def test_linear_bwd_dx_in_place(env):
    """model.mojo:906 calls linear_bwd_dx with grad_input == grad_output."""
    ops, orc, gu = env
    r = gu.rng(3)
    M, C = 512, 256
    dY = gu.randn(r, M, C)
    W = gu.randn(r, C, C, scale=0.05)
    ref = np.zeros((M, C), np.float32)
    orc.call("linear_bwd_dx", ref, dY, W, M, C, C)
    buf = gu.dev(dY)
    ops.linear_bwd_dx(buf, buf, gu.dev(W), M, C, C)
    assert rel_err(gu.host(buf), ref) <= TOL_FP32


@pytest.mark.parametrize("K,N", [(512, 1536), (512, 512), (512, 2048), (2048, 512), (512, 8192)])
def test_gemm_config3_shapes(env, K, N):
    """M = 32768 tokens, bf16 operands, fp32 accumulation,
    against torch fp32 matmul of the same fp32 inputs (tolerance 2e-2)."""
    ops, orc, gu = env
    import torch
    M = 32768
    g = torch.Generator(device="cuda").manual_seed(K + N)
    X = torch.randn(M, K, device="cuda", generator=g)
    W = torch.randn(N, K, device="cuda", generator=g) * 0.02
    dY = torch.randn(M, N, device="cuda", generator=g)
    out = torch.empty(M, N, device="cuda")
    ops.linear_fwd(out, X, W, M, N, K, bf16=True)
    assert rel_err(gu.host(out), gu.host(X @ W.T)) <= TOL_BF16
    dx = torch.empty(M, K, device="cuda")
    ops.linear_bwd_dx(dx, dY, W, M, N, K, bf16=True)
    assert rel_err(gu.host(dx), gu.host(dY @ W)) <= TOL_BF16
    dw = torch.zeros(N, K, device="cuda")
    ops.linear_bwd_dw(dw, dY, X, M, N, K, bf16=True)
    assert rel_err(gu.host(dw), gu.host(dY.T @ X)) <= TOL_BF16
    # fp32 path of the same shape: exact-fp32 matrix cores
    ops.linear_fwd(out, X, W, M, N, K, bf16=False)
    ref = (X.double() @ W.double().T).float()
    assert rel_err(gu.host(out), gu.host(ref)) <= TOL_FP32


@pytest.mark.parametrize("layout", [0, 1, 2])
@pytest.mark.parametrize("M,N,K", [(2048, 768, 512), (1024, 256, 2048), (65536, 512, 512)])
def test_gemm_bf16_storage_persistent(env, layout, M, N, K):
    """bf16 operands in memory at whole-256-tile shapes run the persistent
    direct-to-LDS kernel (the bf16 training step's GEMMs).  Reference: torch
    fp64 matmul of the same bf16 values.  bf16 products are exact in fp32, so
    the fp32-output bound is the accumulation order's (1e-5); bf16 outputs add
    one rounding (2^-9 relative per element, 4e-3 in norm).  Covers NT, NN,
    TN with its reduction split + in-order reduce, and accumulate."""
    ops, orc, gu = env
    import torch
    from autoresearch_amd._lib import check, load
    L = load()
    g = torch.Generator(device="cuda").manual_seed(M + N + K + layout)
    s0 = torch.cuda.current_stream().cuda_stream
    X = (torch.randn(M, N if layout else K, device="cuda", generator=g)).bfloat16()  # X, or dY for NN / TN
    if layout == 2:
        W = torch.randn(M, K, device="cuda", generator=g).bfloat16()                 # the layer input
        ref = X.double().T @ W.double()
        shape = (N, K)
    elif layout == 1:
        W = (torch.randn(N, K, device="cuda", generator=g) * 0.05).bfloat16()
        ref = X.double() @ W.double()
        shape = (M, K)
    else:
        W = (torch.randn(N, K, device="cuda", generator=g) * 0.05).bfloat16()
        ref = X.double() @ W.double().T
        shape = (M, N)
    for c_bf16 in (0, 1):
        C = torch.empty(*shape, device="cuda", dtype=torch.bfloat16 if c_bf16 else torch.float32)
        check(L.ar_gemm_mixed(s0, layout, C.data_ptr(), c_bf16, X.data_ptr(), 1, W.data_ptr(), 1, M, N, K, 0))
        torch.cuda.synchronize()
        tol = 4e-3 if c_bf16 else 1e-5
        assert rel_err(gu.host(C.float()), gu.host(ref.float())) <= tol, (layout, c_bf16)
    # accumulate into an fp32 C that already holds values
    C0 = torch.randn(*shape, device="cuda", generator=g)
    C = C0.clone()
    check(L.ar_gemm_mixed(s0, layout, C.data_ptr(), 0, X.data_ptr(), 1, W.data_ptr(), 1, M, N, K, 1))
    torch.cuda.synchronize()
    assert rel_err(gu.host(C), gu.host((C0.double() + ref).float())) <= 1e-5
    # bit-reproducible: a second call gives the same bits
    C2 = C0.clone()
    check(L.ar_gemm_mixed(s0, layout, C2.data_ptr(), 0, X.data_ptr(), 1, W.data_ptr(), 1, M, N, K, 1))
    torch.cuda.synchronize()
    assert torch.equal(C, C2)


# The dW shapes of BASELINE configs 4 and 5 at their real token counts:
# (M, N, K) of linear_bwd_dw for the fused q|k|v, c_proj, c_fc, mlp_proj and
# lm_head products.  The persistent kernel's reduction split count depends on
# all three, so these are exactly the split counts the benchmark runs.
DW_SHAPES = [(65536, 1536, 512), (65536, 512, 512), (65536, 2048, 512), (65536, 512, 2048), (65536, 8192, 512),
             (131072, 2304, 768), (131072, 768, 768), (131072, 3072, 768), (131072, 768, 3072),
             (131072, 8192, 768)]


@pytest.mark.parametrize("M,N,K", DW_SHAPES)
def test_dw_benchmark_shapes(env, M, N, K):
    """linear_bwd_dw (accumulate) with bf16 operands at the benchmark's shapes
    against torch fp64 of the same bf16 values: products of bf16 values are
    exact in fp32, so the bound is the fp32 accumulation order's (1e-5)."""
    ops, orc, gu = env
    import torch
    from autoresearch_amd._lib import check, load
    L = load()
    g = torch.Generator(device="cuda").manual_seed(M + N + K)
    s0 = torch.cuda.current_stream().cuda_stream
    dY = torch.randn(M, N, device="cuda", generator=g).bfloat16()
    X = torch.randn(M, K, device="cuda", generator=g).bfloat16()
    C0 = torch.randn(N, K, device="cuda", generator=g)
    C = C0.clone()
    check(L.ar_gemm_mixed(s0, 2, C.data_ptr(), 0, dY.data_ptr(), 1, X.data_ptr(), 1, M, N, K, 1))
    ref = C0.double() + dY.double().T @ X.double()
    assert rel_err(gu.host(C), gu.host(ref)) <= 1e-5
    del dY, X, ref
    torch.cuda.empty_cache()


@pytest.mark.parametrize("M,N,K", DW_SHAPES)
def test_dw_benchmark_shapes_fp32(env, M, N, K):
    """linear_bwd_dw (accumulate) with fp32 operands (the fp32 step's dW,
    ops.mojo:953-1033) at the benchmark's shapes against torch fp64 of the
    same values: the north-star fp32 bar 1e-5."""
    ops, orc, gu = env
    import torch
    g = torch.Generator(device="cuda").manual_seed(M + N + K + 1)
    dY = torch.randn(M, N, device="cuda", generator=g)
    X = torch.randn(M, K, device="cuda", generator=g)
    C0 = torch.randn(N, K, device="cuda", generator=g)
    C = C0.clone()
    ops.linear_bwd_dw(C, dY, X, M, N, K)
    ref = C0.double() + dY.double().T @ X.double()
    err = rel_err(gu.host(C), gu.host(ref))
    print(f"MARGIN dw_fp32 M={M} N={N} K={K} rel_err={err:.3e}")
    assert err <= TOL_FP32
    del dY, X, ref
    torch.cuda.empty_cache()


@pytest.mark.parametrize("M", [32768, 200])
def test_lm_head_softcap_ce_config3(env, M):
    """BASELINE config 3's fused LM head: x [M, 512] ~ N(0, 1), lm_head
    [8192, 512] ~ N(0, 0.02^2) as bf16, softcap 15, cross-entropy against
    uniform targets (a few ignored), through ar_lm_head_softcap_ce_bf16 (the
    bf16 step's two launches).  Reference: torch fp64 on the same bf16
    values.  The logits, the loss and the gradient are each one bf16 rounding
    (2^-9 relative) away from it: bounds 4e-3 (logits, gradient, norm-wise)
    and 2e-3 relative on each token's loss, inside the north-star 2e-2."""
    ops, orc, gu = env
    import torch
    from autoresearch_amd._lib import check, load
    L = load()
    V, C, cap, scale = 8192, 512, 15.0, 0.5
    g = torch.Generator(device="cuda").manual_seed(M)
    s0 = torch.cuda.current_stream().cuda_stream
    x = torch.randn(M, C, device="cuda", generator=g).bfloat16()
    w = (torch.randn(V, C, device="cuda", generator=g) * 0.02).bfloat16()
    tg = torch.randint(0, V, (M,), device="cuda", generator=g)
    tg[::97] = -1  # ignored rows
    loss = torch.full((M,), float("nan"), device="cuda")
    logits = torch.empty(M, V, device="cuda", dtype=torch.bfloat16)
    grad = torch.empty(M, V, device="cuda", dtype=torch.bfloat16)
    check(L.ar_lm_head_softcap_ce_bf16(s0, loss.data_ptr(), grad.data_ptr(), logits.data_ptr(), x.data_ptr(),
                                       w.data_ptr(), tg.data_ptr(), M, V, C, cap, scale))
    torch.cuda.synchronize()
    z = x.double() @ w.double().T
    zc = cap * torch.tanh(z / cap)
    live = tg >= 0
    t = tg.clamp(min=0)
    ref_loss = torch.where(live, torch.logsumexp(zc, -1) - zc.gather(1, t[:, None])[:, 0], torch.zeros_like(zc[:, 0]))
    p = torch.softmax(zc, -1)
    p[torch.arange(M, device="cuda"), t] -= 1.0
    ref_grad = torch.where(live[:, None], p * scale, torch.zeros_like(p))
    assert rel_err(gu.host(logits.float()), gu.host(zc)) <= 4e-3
    lg, lr_ = gu.host(loss).astype(np.float64), gu.host(ref_loss)
    assert np.all(np.abs(lg - lr_) <= 2e-3 * np.abs(lr_)), np.abs(lg - lr_).max()
    assert np.all(lg[::97] == 0.0)
    assert rel_err(gu.host(grad.float()), gu.host(ref_grad)) <= 4e-3
    assert torch.all(grad[::97] == 0)
    # the per-row gradient sums to 0 (softmax sums to 1) up to the bf16 rounding
    rs = grad.float().sum(-1)
    assert float(rs.abs().max()) <= 4e-3 * scale  # the -1 entry alone rounds by up to 2^-10


def _attn_inputs(gu, r, B, T, H, hd):
    q = gu.randn(r, B, T, H, hd)
    k = gu.randn(r, B, T, H, hd)
    v = gu.randn(r, B, T, H, hd)
    do = gu.randn(r, B, T, H, hd)
    return q, k, v, do


# hd 16 / 80 / 96 / 100 / 7 run the tiled kernels on zero-padded rows
# (ops.mojo:267 accepts any head_dim <= 128); (1, 200, 2, 128, 50) runs
# partial 32- and 64-row tiles at hd 128.
@pytest.mark.parametrize("B,T,H,hd,window", [(1, 128, 2, 64, 0), (2, 200, 2, 64, 32), (1, 256, 4, 128, 0),
                                              (1, 320, 1, 128, 100), (2, 64, 2, 32, 16), (1, 200, 2, 128, 50),
                                              (2, 96, 2, 16, 0), (1, 150, 3, 80, 40), (1, 128, 2, 96, 0),
                                              (2, 70, 1, 100, 20), (1, 33, 2, 7, 0)])
@pytest.mark.parametrize("bf16", [False, True])
def test_attention_vs_oracle(env, B, T, H, hd, window, bf16):
    ops, orc, gu = env
    r = gu.rng(T + hd + window)
    tol = TOL_BF16 if bf16 else TOL_FP32
    q, k, v, do = _attn_inputs(gu, r, B, T, H, hd)
    n = B * T * H
    o_ref, lse_ref = np.zeros_like(q), np.zeros(n, np.float32)
    orc.call("flash_attn_fwd", o_ref, lse_ref, q, k, v, B, T, H, hd, window)
    d_ref = np.zeros(n, np.float32)
    orc.call("flash_attn_bwd_precompute_d", d_ref, o_ref, do, B, T, H, hd)
    dq_ref = np.zeros_like(q)
    orc.call("flash_attn_bwd_dq", dq_ref, q, k, v, do, lse_ref, d_ref, B, T, H, hd, window)
    dk_ref, dv_ref = np.zeros_like(q), np.zeros_like(q)
    orc.call("flash_attn_bwd_dkv", dk_ref, dv_ref, q, k, v, do, lse_ref, d_ref, B, T, H, hd, window)

    qd, kd, vd, dod = gu.dev(q), gu.dev(k), gu.dev(v), gu.dev(do)
    o, lse = gu.empty(B, T, H, hd), gu.empty(n)
    ops.flash_attn_fwd(o, lse, qd, kd, vd, B, T, H, hd, window, bf16=bf16)
    assert rel_err(gu.host(o), o_ref) <= tol
    assert rel_err(gu.host(lse), lse_ref) <= (tol if not bf16 else 1e-2)
    # backward from the oracle's forward statistics, so each kernel is checked alone
    lse_d, d_d = gu.dev(lse_ref), gu.dev(d_ref)
    dq = gu.empty(B, T, H, hd)
    ops.flash_attn_bwd_dq(dq, qd, kd, vd, dod, lse_d, d_d, B, T, H, hd, window, bf16=bf16)
    assert rel_err(gu.host(dq), dq_ref) <= tol
    dk, dv = gu.empty(B, T, H, hd), gu.empty(B, T, H, hd)
    ops.flash_attn_bwd_dkv(dk, dv, qd, kd, vd, dod, lse_d, d_d, B, T, H, hd, window, bf16=bf16)
    assert rel_err(gu.host(dk), dk_ref) <= tol
    assert rel_err(gu.host(dv), dv_ref) <= tol


def _torch_attention(q, k, v, window):
    """fp32 masked softmax attention on the GPU (math path), [B,T,H,hd]."""
    import torch
    B, T, H, hd = q.shape
    qt, kt, vt = (x.permute(0, 2, 1, 3).contiguous() for x in (q, k, v))
    s = torch.matmul(qt, kt.transpose(-1, -2).contiguous()) / np.sqrt(hd)
    i = torch.arange(T, device=q.device)
    vis = i[None, :] <= i[:, None]
    if window > 0:
        vis &= i[None, :] >= i[:, None] - window
    s = s.masked_fill(~vis, float("-inf"))
    lse = torch.logsumexp(s, -1)
    o = torch.matmul(torch.softmax(s, -1), vt)
    return o.permute(0, 2, 1, 3).contiguous(), lse.permute(0, 2, 1).contiguous()


@pytest.mark.parametrize("window", [0, 1024])
@pytest.mark.parametrize("bf16", [False, True])
def test_attention_config2(env, window, bf16):
    """B16 H4 hd128 T2048, RoPE'd q/k, full causal and
    window 1024; forward against torch fp32, backward via autograd of the same
    torch reference (fp32 tolerance 1e-5 / bf16 2e-2)."""
    ops, orc, gu = env
    import torch
    B, T, H, hd = 16, 2048, 4, 128
    g = torch.Generator(device="cuda").manual_seed(7 + window)
    q, k, v, do = (torch.randn(B, T, H, hd, device="cuda", generator=g) for _ in range(4))
    # RoPE (base 10000, per-sequence positions) on q and k, as the config states
    c = torch.empty(T * hd // 2, device="cuda")
    s = torch.empty(T * hd // 2, device="cuda")
    ops.precompute_rope(c, s, T, hd)
    for b in range(B):
        for x in (q, k):
            xb = x[b].contiguous()
            ops.rope_fwd(xb, xb, c, s, T, H, hd)
            x[b].copy_(xb)
    tol = TOL_BF16 if bf16 else TOL_FP32
    n = B * T * H
    o, lse = torch.empty_like(q), torch.empty(n, device="cuda")
    ops.flash_attn_fwd(o, lse, q, k, v, B, T, H, hd, window, bf16=bf16)
    with torch.no_grad():
        o_ref, lse_ref = _torch_attention(q, k, v, window)
    assert rel_err(gu.host(o), gu.host(o_ref)) <= tol
    assert rel_err(gu.host(lse), gu.host(lse_ref)) <= tol
    dbuf = torch.empty(n, device="cuda")
    ops.flash_attn_bwd_precompute_d(dbuf, o, do, B, T, H, hd, bf16=bf16)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    ops.flash_attn_bwd_dq(dq, q, k, v, do, lse, dbuf, B, T, H, hd, window, bf16=bf16)
    ops.flash_attn_bwd_dkv(dk, dv, q, k, v, do, lse, dbuf, B, T, H, hd, window, bf16=bf16)
    qr, kr, vr = (x.clone().requires_grad_(True) for x in (q, k, v))
    o2, _ = _torch_attention(qr, kr, vr, window)
    o2.backward(do)
    assert rel_err(gu.host(dq), gu.host(qr.grad)) <= tol
    assert rel_err(gu.host(dk), gu.host(kr.grad)) <= tol
    assert rel_err(gu.host(dv), gu.host(vr.grad)) <= tol


# (30, 50), (50, 30), (13, 7), (100, 100): shapes that are not multiples of 8
# (optimizer.mojo:255-342 takes any matrix)
@pytest.mark.parametrize("rows,cols", [(128, 128), (512, 128), (128, 512), (256, 1024), (30, 50), (50, 30), (13, 7),
                                       (100, 100)])
@pytest.mark.parametrize("bf16", [False, True])
def test_muon_step_vs_oracle(env, rows, cols, bf16):
    ops, orc, gu = env
    r = gu.rng(rows * 3 + cols)
    p = gu.randn(r, rows, cols, scale=0.05)
    g = gu.randn(r, rows, cols, scale=0.01)
    mb = gu.randn(r, rows, cols, scale=0.01)
    p_ref, g_ref, mb_ref = p.copy(), g.copy(), mb.copy()
    orc.call("muon_step", p_ref, g_ref, mb_ref, rows, cols, 0.04, 1.0, 0.85, 0.2)
    pd, gd, mbd = gu.dev(p), gu.dev(g), gu.dev(mb)
    ops.muon_step(pd, gd, mbd, rows, cols, 0.04, 1.0, 0.85, 0.2, bf16=bf16)
    assert rel_err(gu.host(mbd), mb_ref) <= TOL_FP32
    # post-step weights: the north-star bar (fp32 1e-5, bf16 2e-2)
    assert rel_err(gu.host(pd), p_ref) <= (TOL_BF16 if bf16 else TOL_FP32)
    # the applied update p_new - p itself, after five Polar Express
    # iterations whose polynomial amplifies operand rounding: fp32 <= 1e-4,
    # bf16 operands <= 6e-2 (bf16-operand Muon is the reference design's
    # intent; the fp32 oracle is the comparison point)
    upd, upd_ref = gu.host(pd) - p, p_ref - p
    assert rel_err(upd, upd_ref) <= (6e-2 if bf16 else 1e-4)
