"""Per-op parity: every C-ABI kernel entry point against the CPU oracle on the
same seeded inputs (fp32 rel-err <= 1e-5, bf16 <= 2e-2, gather/scatter
bit-exact).  Runs on the GPU through autoresearch_amd.ops (the C ABI)."""
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


def test_embedding_fwd_bitexact(env):
    ops, orc, gu = env
    r = gu.rng(1)
    V, D, n = 97, 520, 1000
    w = gu.randn(r, V, D)
    idx = r.integers(0, V, n).astype(np.int64)
    ref = np.zeros((n, D), np.float32)
    orc.call("embedding_fwd", ref, w, idx, n, D)
    out = gu.empty(n, D)
    ops.embedding_fwd(out, gu.dev(w), gu.dev(idx), n, D)
    np.testing.assert_array_equal(gu.host(out), ref)


def test_embedding_kat(env):
    """test_kernels.mojo:20-64: W[v,d] = 10v + d, idx [2,5,0]."""
    ops, orc, gu = env
    w = np.array([[10 * v + d for d in range(4)] for v in range(8)], np.float32)
    idx = np.array([2, 5, 0], np.int64)
    out = gu.empty(3, 4)
    ops.embedding_fwd(out, gu.dev(w), gu.dev(idx), 3, 4)
    np.testing.assert_array_equal(gu.host(out), [[20, 21, 22, 23], [50, 51, 52, 53], [0, 1, 2, 3]])


@pytest.mark.parametrize("n,dim,zipf", [(4096, 512, True), (333, 128, False), (64, 40, False), (65536, 512, True),
                                         (20000, 768, True), (3000, 1024, True), (500, 1000, False)])
def test_embedding_bwd_bitexact(env, n, dim, zipf):
    ops, orc, gu = env
    r = gu.rng(2)
    V = 300
    if zipf:
        p = 1.0 / np.arange(1, V + 1) ** 1.1
        idx = r.choice(V, size=n, p=p / p.sum()).astype(np.int64)
    else:
        idx = r.integers(0, V, n).astype(np.int64)
    g0 = gu.randn(r, V, dim)
    dy = gu.randn(r, n, dim)
    ref = g0.copy()
    orc.call("embedding_bwd", ref, dy, idx, n, dim)
    gw = gu.dev(g0)
    ops.embedding_bwd(gw, gu.dev(dy), gu.dev(idx), n, dim)
    np.testing.assert_array_equal(gu.host(gw), ref)
    # run-to-run determinism
    gw2 = gu.dev(g0)
    ops.embedding_bwd(gw2, gu.dev(dy), gu.dev(idx), n, dim)
    np.testing.assert_array_equal(gu.host(gw2), gu.host(gw))


@pytest.mark.parametrize("rows,dim", [(2, 4), (1000, 512), (4096, 128), (77, 64)])
def test_rmsnorm_fwd_bwd(env, rows, dim):
    ops, orc, gu = env
    r = gu.rng(3)
    x = gu.randn(r, rows, dim, scale=2.0)
    dy = gu.randn(r, rows, dim)
    y_ref = np.zeros_like(x)
    rms_ref = np.zeros(rows, np.float32)
    orc.call("rmsnorm_fwd", y_ref, rms_ref, x, rows, dim)
    dx_ref = np.zeros_like(x)
    orc.call("rmsnorm_bwd", dx_ref, dy, x, rms_ref, rows, dim)
    xd = gu.dev(x)
    y = gu.empty(rows, dim)
    rms = gu.empty(rows)
    ops.rmsnorm_fwd(y, rms, xd, rows, dim)
    assert rel_err(gu.host(y), y_ref) <= TOL_FP32
    assert rel_err(gu.host(rms), rms_ref) <= TOL_FP32
    # in place (model.mojo:612) and in-place backward (model.mojo:858)
    ops.rmsnorm_fwd(xd, rms, xd, rows, dim)
    assert rel_err(gu.host(xd), y_ref) <= TOL_FP32
    g = gu.dev(dy)
    ops.rmsnorm_bwd(g, g, gu.dev(x), gu.dev(rms_ref), rows, dim)
    assert rel_err(gu.host(g), dx_ref) <= TOL_FP32


def test_rmsnorm_kat(env):
    """test_kernels.mojo:140-181"""
    ops, orc, gu = env
    x = np.array([[1, 2, 3, 4], [0, 0, 0, 5]], np.float32)
    y, rms = gu.empty(2, 4), gu.empty(2)
    ops.rmsnorm_fwd(y, rms, gu.dev(x), 2, 4)
    rh, yh = gu.host(rms), gu.host(y)
    assert abs(rh[0] - 2.7386) < 0.01 and abs(rh[1] - 2.5) < 0.01
    assert abs(yh[0, 0] - 1 / 2.7386) < 0.01 and abs(yh[1, 3] - 2.0) < 0.01


def _rope_tables(orc, rows, hd):
    c = np.zeros((rows, hd // 2), np.float32)
    s = np.zeros_like(c)
    orc.call("precompute_rope", c, s, rows, hd, 10000.0)
    return c, s


@pytest.mark.parametrize("nt,H,hd", [(256, 4, 128), (128, 2, 64)])
def test_rope_fwd_bwd(env, nt, H, hd):
    ops, orc, gu = env
    r = gu.rng(4)
    c, s = _rope_tables(orc, nt, hd)
    x = gu.randn(r, nt, H, hd)
    ref = np.zeros_like(x)
    orc.call("rope_fwd", ref, x, c, s, nt, H, hd)
    refb = np.zeros_like(x)
    orc.call("rope_bwd", refb, x, c, s, nt, H, hd)
    xd = gu.dev(x)
    cd, sd = gu.dev(c), gu.dev(s)
    ops.rope_fwd(xd, xd, cd, sd, nt, H, hd)  # in place, as model.mojo:668
    assert rel_err(gu.host(xd), ref) <= TOL_FP32
    xb = gu.dev(x)
    ops.rope_bwd(xb, xb, cd, sd, nt, H, hd)
    assert rel_err(gu.host(xb), refb) <= TOL_FP32


def test_precompute_rope(env):
    ops, orc, gu = env
    import torch
    c_ref, s_ref = _rope_tables(orc, 2048, 128)
    c = torch.empty(2048 * 64, device="cuda")
    s = torch.empty(2048 * 64, device="cuda")
    ops.precompute_rope(c, s, 2048, 128)
    np.testing.assert_array_equal(gu.host(c).reshape(2048, 64), c_ref)
    np.testing.assert_array_equal(gu.host(s).reshape(2048, 64), s_ref)


def test_elementwise(env):
    ops, orc, gu = env
    r = gu.rng(5)
    n = 100003  # odd size: exercises the scalar path
    for size in (n, 1 << 16):
        x = gu.randn(r, size, scale=3.0)
        y = gu.randn(r, size)
        ref = np.zeros_like(x)
        out = gu.empty(size)
        orc.call("relu_squared_fwd", ref, x, size)
        ops.relu_squared_fwd(out, gu.dev(x), size)
        assert rel_err(gu.host(out), ref) <= TOL_FP32
        orc.call("relu_squared_bwd", ref, y, x, size)
        ops.relu_squared_bwd(out, gu.dev(y), gu.dev(x), size)
        assert rel_err(gu.host(out), ref) <= TOL_FP32
        xs = x * 20
        orc.call("softcap_fwd", ref, xs, 15.0, size)
        ops.softcap_fwd(out, gu.dev(xs), 15.0, size)
        assert rel_err(gu.host(out), ref) <= TOL_FP32
        orc.call("add_residual_fwd", ref, x, y, size)
        xd = gu.dev(x)
        ops.add_residual_fwd(xd, xd, gu.dev(y), size)
        np.testing.assert_array_equal(gu.host(xd), ref)
        sa = np.array([0.5, 1.25], np.float32)
        sb = np.array([0.1, -0.3], np.float32)
        orc.call("scaled_add_fwd", ref, x, y, sa, sb, 1, size)
        ops.scaled_add_fwd(out, gu.dev(x), gu.dev(y), gu.dev(sa), gu.dev(sb), 1, size)
        assert rel_err(gu.host(out), ref) <= TOL_FP32
        ga, gb = np.zeros_like(x), np.zeros_like(x)
        orc.call("scaled_add_bwd", ga, gb, x, sa, sb, 1, size)
        gad, gbd = gu.dev(x), gu.empty(size)
        ops.scaled_add_bwd(gad, gbd, gad, gu.dev(sa), gu.dev(sb), 1, size)  # model.mojo:1020 aliasing
        np.testing.assert_array_equal(gu.host(gad), ga)
        np.testing.assert_array_equal(gu.host(gbd), gb)
        orc.call("scale_add", ref, x, y, -1.5, 0.75, size)
        ops.scale_add_kernel(out, gu.dev(x), gu.dev(y), -1.5, 0.75, size)
        assert rel_err(gu.host(out), ref) <= TOL_FP32
        ops.zero_buffer(out, size)
        assert np.all(gu.host(out) == 0)


def test_softcap_kat(env):
    """test_kernels.mojo:103-137"""
    ops, orc, gu = env
    x = np.array([0.0, 15.0, -30.0, 100.0], np.float32)
    out = gu.empty(4)
    ops.softcap_fwd(out, gu.dev(x), 15.0, 4)
    o = gu.host(out)
    assert abs(o[0]) <= 1e-5 and abs(o[3] - 15.0) <= 0.1 and o[2] < -14.0


def test_relu2_kat(env):
    """test_kernels.mojo:67-100"""
    ops, orc, gu = env
    x = np.array([-2, -1, 0, 1, 2, 3], np.float32)
    out = gu.empty(6)
    ops.relu_squared_fwd(out, gu.dev(x), 6)
    np.testing.assert_allclose(gu.host(out), [0, 0, 0, 1, 4, 9], atol=1e-5)


@pytest.mark.parametrize("nt,V", [(2, 4), (300, 8192), (64, 512)])
def test_cross_entropy(env, nt, V):
    ops, orc, gu = env
    r = gu.rng(6)
    logits = gu.randn(r, nt, V, scale=4.0)
    tg = r.integers(0, V, nt).astype(np.int64)
    tg[0] = -1  # ignored target
    loss_ref = np.zeros(nt, np.float32)
    orc.call("cross_entropy_fwd", loss_ref, logits, tg, nt, V)
    loss = gu.empty(nt)
    ops.cross_entropy_fwd(loss, gu.dev(logits), gu.dev(tg), nt, V)
    assert rel_err(gu.host(loss), loss_ref) <= TOL_FP32
    assert gu.host(loss)[0] == 0.0
    g_ref = np.zeros_like(logits)
    orc.call("cross_entropy_softcap_bwd", g_ref, logits, tg, 15.0, nt, V, 0.5)
    g = gu.empty(nt, V)
    ops.cross_entropy_softcap_bwd(g, gu.dev(logits), gu.dev(tg), 15.0, nt, V, 0.5)
    assert rel_err(gu.host(g), g_ref) <= TOL_FP32
    m_ref = np.zeros(1, np.float32)
    orc.call("mean_reduce", m_ref, loss_ref, nt)
    m = gu.empty(1)
    ops.mean_reduce(m, gu.dev(loss_ref), nt)
    assert rel_err(gu.host(m), m_ref) <= TOL_FP32


def test_cross_entropy_kat(env):
    """test_kernels.mojo:227-267"""
    ops, orc, gu = env
    logits = np.array([[1, 2, 3, 4], [4, 3, 2, 1]], np.float32)
    tg = np.array([3, 3], np.int64)
    loss = gu.empty(2)
    ops.cross_entropy_fwd(loss, gu.dev(logits), gu.dev(tg), 2, 4)
    lh = gu.host(loss)
    assert abs(lh[0] - 0.4402) < 0.01 and abs(lh[1] - 3.4402) < 0.01


def test_softmax(env):
    ops, orc, gu = env
    r = gu.rng(7)
    x = gu.randn(r, 33, 1000)
    out = gu.empty(33, 1000)
    ops.softmax_fwd(out, gu.dev(x), 33, 1000)
    ex = np.exp(x.astype(np.float64) - x.max(1, keepdims=True))
    assert rel_err(gu.host(out), ex / ex.sum(1, keepdims=True)) <= TOL_FP32


@pytest.mark.parametrize("nt,gc", [(512, 32), (3001, 48), (70000, 32)])
def test_ve_kernels(env, nt, gc):
    ops, orc, gu = env
    r = gu.rng(8)
    H, hd = 4, 128
    C = H * hd
    xn = gu.randn(r, nt, C)
    w = gu.randn(r, H, gc, scale=0.2)
    gate_ref = np.zeros((nt, H), np.float32)
    orc.call("ve_gate_fwd", gate_ref, xn, w, nt, H, gc, C)
    gate = gu.empty(nt, H)
    ops.ve_gate_fwd(gate, gu.dev(xn), gu.dev(w), nt, H, gc, C)
    assert rel_err(gu.host(gate), gate_ref) <= TOL_FP32
    v = gu.randn(r, nt, H, hd)
    ve = gu.randn(r, nt, H, hd)
    v_ref = v.copy()
    orc.call("ve_apply_fwd", v_ref, gate_ref, ve, nt, H, hd)
    vd = gu.dev(v)
    ops.ve_apply_fwd(vd, gu.dev(gate_ref), gu.dev(ve), nt, H, hd)
    assert rel_err(gu.host(vd), v_ref) <= TOL_FP32
    gv = gu.randn(r, nt, H, hd)
    gve_ref, gg_ref = np.zeros_like(gv), np.zeros((nt, H), np.float32)
    orc.call("ve_apply_bwd", gve_ref, gg_ref, gv, gate_ref, ve, nt, H, hd)
    gve, gg = gu.empty(nt, H, hd), gu.empty(nt, H)
    ops.ve_apply_bwd(gve, gg, gu.dev(gv), gu.dev(gate_ref), gu.dev(ve), nt, H, hd)
    assert rel_err(gu.host(gve), gve_ref) <= TOL_FP32
    assert rel_err(gu.host(gg), gg_ref) <= TOL_FP32
    gx0 = gu.randn(r, nt, C)
    gw0 = gu.randn(r, H, gc)
    gx_ref, gw_ref = gx0.copy(), gw0.copy()
    orc.call("ve_gate_bwd", gx_ref, gw_ref, gg_ref, gate_ref, xn, w, nt, H, gc, C)
    gx, gw = gu.dev(gx0), gu.dev(gw0)
    ops.ve_gate_bwd(gx, gw, gu.dev(gg_ref), gu.dev(gate_ref), gu.dev(xn), gu.dev(w), nt, H, gc, C)
    assert rel_err(gu.host(gx), gx_ref) <= TOL_FP32
    assert rel_err(gu.host(gw), gw_ref) <= TOL_FP32


def test_scalar_grad_reduce(env):
    ops, orc, gu = env
    r = gu.rng(9)
    n = 1 << 20
    g, x = gu.randn(r, n), gu.randn(r, n)
    gs0 = np.array([0.5, -2.0, 3.0], np.float32)
    ref = gs0.copy()
    orc.call("scalar_grad_reduce", ref, g, x, 2, n)
    gs = gu.dev(gs0)
    ops.scalar_grad_reduce(gs, gu.dev(g), gu.dev(x), 2, n)
    h = gu.host(gs)
    assert np.array_equal(h[:2], gs0[:2])
    assert abs(h[2] - ref[2]) <= TOL_FP32 * max(1.0, np.sqrt(n))


def test_precompute_d(env):
    ops, orc, gu = env
    r = gu.rng(10)
    B, T, H, hd = 2, 64, 4, 128
    o, g = gu.randn(r, B * T * H, hd), gu.randn(r, B * T * H, hd)
    ref = np.zeros(B * T * H, np.float32)
    orc.call("flash_attn_bwd_precompute_d", ref, o, g, B, T, H, hd)
    d = gu.empty(B * T * H)
    ops.flash_attn_bwd_precompute_d(d, gu.dev(o), gu.dev(g), B, T, H, hd)
    assert rel_err(gu.host(d), ref) <= TOL_FP32


def test_optimizer_kernels(env):
    ops, orc, gu = env
    r = gu.rng(11)
    n = 50000
    p, g = gu.randn(r, n), gu.randn(r, n, scale=0.1)
    m, v = gu.randn(r, n, scale=0.01), np.abs(gu.randn(r, n, scale=0.01))
    refs = [a.copy() for a in (p, g, m, v)]
    orc.call("adamw", refs[0], refs[1], refs[2], refs[3], 0.01, 0.8, 0.95, 1e-10, 0.1, 0.36, 0.0975, n)
    ds = [gu.dev(a) for a in (p, g, m, v)]
    ops.adamw_kernel(ds[0], ds[1], ds[2], ds[3], 0.01, 0.8, 0.95, 1e-10, 0.1, 0.36, 0.0975, n)
    for d_, r_ in zip(ds, refs):
        assert rel_err(gu.host(d_), r_) <= TOL_FP32
    out_ref, buf_ref = np.zeros_like(p), m.copy()
    orc.call("nesterov_momentum", out_ref, g, buf_ref, 0.9, n)
    out, buf = gu.empty(n), gu.dev(m)
    ops.nesterov_momentum_kernel(out, gu.dev(g), buf, 0.9, n)
    assert rel_err(gu.host(out), out_ref) <= TOL_FP32
    assert rel_err(gu.host(buf), buf_ref) <= TOL_FP32
    x_ref = p.copy()
    orc.call("normalize_frobenius", x_ref, n)
    xd = gu.dev(p)
    ops.normalize_frobenius_kernel(xd, n)
    assert rel_err(gu.host(xd), x_ref) <= TOL_FP32
    pr = p.copy()
    orc.call("muon_update", pr, g, 0.02, 0.2, n)
    pd = gu.dev(p)
    ops.muon_update_kernel(pd, gu.dev(g), 0.02, 0.2, n)
    assert rel_err(gu.host(pd), pr) <= TOL_FP32


def test_init_kernels(env):
    ops, orc, gu = env
    import torch
    n = 123457
    ref = np.zeros(n, np.float32)
    out = torch.empty(n, device="cuda")
    orc.call("fill_uniform", ref, 45, -0.0765, 0.0765, n)
    ops.fill_uniform_kernel(out, 45, -0.0765, 0.0765, n)
    np.testing.assert_array_equal(gu.host(out), ref)  # bit-exact
    orc.call("fill_normal", ref, 42, 1.0, n)
    ops.fill_normal_kernel(out, 42, 1.0, n)
    # GPU logf/cosf/sqrtf vs glibc: a few ulp, far inside the fp32 bar
    assert rel_err(gu.host(out), ref) <= TOL_FP32
    ops.fill_value_kernel(out, 0.1, n)
    assert np.all(gu.host(out) == np.float32(0.1))
    ops.fill_zeros_kernel(out, n)
    assert np.all(gu.host(out) == 0)


def test_errors(env):
    ops, orc, gu = env
    from autoresearch_amd._lib import ArError
    import torch
    q = torch.zeros(2 * 16 * 1 * 256, device="cuda")
    with pytest.raises(ArError):
        ops.flash_attn_fwd(q, torch.zeros(32, device="cuda"), q, q, q, 2, 16, 1, 256, 0)  # hd > 128 (ops.mojo:267)
    a = torch.zeros(24, device="cuda")
    with pytest.raises(ArError, match="overlaps"):
        ops.linear_fwd(a, a, a, 3, 4, 2)  # the output aliases an input
    with pytest.raises(ArError, match="negative"):
        ops.linear_fwd(torch.zeros(24, device="cuda"), a, a, -3, 4, 2)


def _sort_fn():
    """ar_embedding_sort (the embedding scatter's stable token sort; declared
    for the library's own callers, not in the public header)."""
    import ctypes as ct
    from autoresearch_amd._lib import load
    fn = load().ar_embedding_sort
    fn.restype = ct.c_int32
    fn.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_void_p, ct.c_void_p, ct.c_int64, ct.c_int32, ct.c_void_p,
                   ct.c_size_t, ct.POINTER(ct.c_size_t)]
    return fn


@pytest.mark.parametrize("n,end_bit,dist", [(1, 13, "u"), (63, 13, "u"), (64, 7, "u"), (2049, 13, "zipf"),
                                            (65536, 13, "zipf"), (131072, 13, "zipf"), (100003, 32, "u"),
                                            (4096, 32, "same")])
def test_embedding_sort_stable(env, n, end_bit, dist):
    """The hand-written counting sort: ids ascending, equal ids in token order
    (exactly numpy's stable argsort), for one to three digit passes, partial
    tiles and rounds, Zipf-hot ids, and all-equal ids."""
    ops, orc, gu = env
    import ctypes as ct
    import torch
    from autoresearch_amd._lib import check
    r = gu.rng(n + end_bit)
    hi = min(1 << end_bit, 1 << 31)
    if dist == "zipf":
        V = min(hi, 8192)
        p = 1.0 / np.arange(1, V + 1) ** 1.1
        idx = r.choice(V, size=n, p=p / p.sum()).astype(np.int64)
    elif dist == "same":
        idx = np.full(n, 77, np.int64)
    else:
        idx = r.integers(0, hi, n).astype(np.int64)
    fn = _sort_fn()
    need = ct.c_size_t()
    check(fn(None, None, None, None, n, end_bit, None, 0, ct.byref(need)), "embedding_sort")
    scratch = torch.empty(need.value, dtype=torch.uint8, device="cuda")
    sid = torch.empty(n, dtype=torch.int32, device="cuda")
    stok = torch.empty(n, dtype=torch.int32, device="cuda")
    d_idx = gu.dev(idx)
    s0 = torch.cuda.current_stream().cuda_stream
    check(fn(s0, sid.data_ptr(), stok.data_ptr(), d_idx.data_ptr(), n, end_bit, scratch.data_ptr(), need.value, None),
          "embedding_sort")
    order = np.argsort(idx, kind="stable")
    np.testing.assert_array_equal(gu.host(stok), order.astype(np.int32))
    np.testing.assert_array_equal(gu.host(sid).view(np.uint32), idx[order].astype(np.uint32))


def test_workspace_binding_errors(env):
    """A per-op call that needs scratch fails (AR_ENOMEM, naming the bytes)
    on a stream with no workspace or too small a one, and allocates nothing."""
    ops, orc, gu = env
    import torch
    from autoresearch_amd._lib import ArError
    M, N, K = 4096, 512, 512
    dY, X = torch.randn(M, N, device="cuda"), torch.randn(M, K, device="cuda")
    dw = torch.zeros(N, K, device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with pytest.raises(ArError, match="no workspace bound"):
            ops.linear_bwd_dw(dw, dY, X, M, N, K)
        small = ops.Workspace(4096).bind()
        with pytest.raises(ArError, match="needs"):
            ops.linear_bwd_dw(dw, dY, X, M, N, K)
        big = ops.Workspace(64 << 20).bind()  # rebinding replaces the small one
        ops.linear_bwd_dw(dw, dY, X, M, N, K)
        s.synchronize()
        small.close()
        big.close()
        with pytest.raises(ArError, match="no workspace bound"):
            ops.linear_bwd_dw(dw, dY, X, M, N, K)
    ref = dY.double().T @ X.double()
    assert rel_err(gu.host(dw), gu.host(ref)) <= TOL_FP32


def test_per_op_calls_under_stream_capture(env):
    """Per-op entry points that use scratch (split-K dW partials + reduce, the
    embedding sort + chunk sums, a multi-block mean) record into a graph: no
    allocation or synchronisation happens inside them.  The graph is replayed
    five times with eager work in between, each replay checked bit for bit
    against the eager result."""
    ops, orc, gu = env
    import torch
    r = gu.rng(11)
    M, N, K, V = 8192, 512, 512, 1000
    dY, X = gu.dev(gu.randn(r, M, N)), gu.dev(gu.randn(r, M, K))
    idx = gu.dev(r.integers(0, V, M).astype(np.int64))
    dw0, gw0 = gu.dev(gu.randn(r, N, K)), gu.dev(gu.randn(r, V, N))
    loss = gu.dev(gu.randn(r, M))
    s = torch.cuda.Stream()
    ws = ops.Workspace(256 << 20).bind(s)
    dw, gw, mean = dw0.clone(), gw0.clone(), torch.zeros(1, device="cuda")

    def body():
        ops.linear_bwd_dw(dw, dY, X, M, N, K)
        ops.embedding_bwd(gw, dY, idx, M, N)
        ops.mean_reduce(mean, loss, M)

    with torch.cuda.stream(s):
        body()
    s.synchronize()
    want = (gu.host(dw).copy(), gu.host(gw).copy(), gu.host(mean).copy())
    g = torch.cuda.CUDAGraph()
    dw.copy_(dw0)
    gw.copy_(gw0)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        body()
    for rep in range(5):
        dw.copy_(dw0)
        gw.copy_(gw0)
        mean.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(gu.host(dw), want[0], err_msg=f"replay {rep}")
        np.testing.assert_array_equal(gu.host(gw), want[1], err_msg=f"replay {rep}")
        np.testing.assert_array_equal(gu.host(mean), want[2], err_msg=f"replay {rep}")
        _ = (dY * 2).sum()  # eager work between replays
    del g
    ws.close()
