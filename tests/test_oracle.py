"""Pins the CPU oracle (oracle/ar_oracle.c) before it is trusted as the parity
checker: the reference's own known-answer tests (test_kernels.mojo), fp64
numpy / torch-CPU autograd for the closed-form ops, torch's AdamW, invariants
of the Polar Express orthogonalisation, an independent uint64 restatement of
the init PRNG, and whole-model behaviour from test_forward.mojo /
test_backward.mojo.  CPU only."""
import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------- reference KATs (test_kernels.mojo) ----------------
def _kats():
    with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
        return json.load(f)


def test_kat_embedding():
    k = _kats()["embedding"]
    w = f32(k["weight"])
    idx = np.array(k["indices"], np.int64)
    out = np.zeros((len(idx), w.shape[1]), np.float32)
    orc.call("embedding_fwd", out, w, idx, len(idx), w.shape[1])
    np.testing.assert_array_equal(out, k["expected"])


def test_kat_relu_squared():
    k = _kats()["relu_squared"]
    x = f32(k["input"])
    out = np.zeros_like(x)
    orc.call("relu_squared_fwd", out, x, x.size)
    assert np.all(np.abs(out - k["expected"]) <= k["atol"])


def test_kat_softcap():
    k = _kats()["softcap"]
    x = f32(k["input"])
    out = np.zeros_like(x)
    orc.call("softcap_fwd", out, x, k["cap"], x.size)
    assert abs(out[0]) <= 1e-5 and abs(out[3] - 15.0) <= 0.1 and out[2] < -14.0


def test_kat_rmsnorm():
    k = _kats()["rmsnorm"]
    x = f32(k["input"])
    out, rms = np.zeros_like(x), np.zeros(x.shape[0], np.float32)
    orc.call("rmsnorm_fwd", out, rms, x, x.shape[0], x.shape[1])
    assert np.all(np.abs(rms - k["rms"]) <= k["atol"])
    assert abs(out[0, 0] - k["out00"]) <= k["atol"] and abs(out[1, 3] - k["out13"]) <= k["atol"]


def test_kat_cross_entropy():
    k = _kats()["cross_entropy"]
    logits = f32(k["logits"])
    tg = np.array(k["targets"], np.int64)
    loss = np.zeros(2, np.float32)
    orc.call("cross_entropy_fwd", loss, logits, tg, 2, 4)
    assert np.all(np.abs(loss - k["expected"]) <= k["atol"]) and loss[0] < loss[1]


# ---------------- closed forms vs fp64 ----------------
def test_rmsnorm_vs_autograd():
    r = np.random.default_rng(0)
    x = f32(r.standard_normal((37, 96)) * 3)
    dy = f32(r.standard_normal((37, 96)))
    out, rms = np.zeros_like(x), np.zeros(37, np.float32)
    orc.call("rmsnorm_fwd", out, rms, x, 37, 96)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    rt = torch.sqrt((xt * xt).mean(1, keepdim=True) + 1e-5)
    yt = xt / rt
    yt.backward(torch.tensor(dy, dtype=torch.float64))
    np.testing.assert_allclose(out, yt.detach().numpy(), rtol=2e-6, atol=1e-6)
    np.testing.assert_allclose(rms, rt.detach().numpy().ravel(), rtol=2e-6)
    dx = np.zeros_like(x)
    orc.call("rmsnorm_bwd", dx, dy, x, rms, 37, 96)
    np.testing.assert_allclose(dx, xt.grad.numpy(), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("M,N,K", [(13, 24, 40), (64, 8, 200)])
def test_linear_layouts_vs_numpy(M, N, K):
    r = np.random.default_rng(M)
    X, W, dY = f32(r.standard_normal((M, K))), f32(r.standard_normal((N, K))), f32(r.standard_normal((M, N)))
    X64, W64, dY64 = X.astype(np.float64), W.astype(np.float64), dY.astype(np.float64)
    y = np.zeros((M, N), np.float32)
    orc.call("linear_fwd", y, X, W, M, N, K)
    np.testing.assert_allclose(y, X64 @ W64.T, rtol=1e-6, atol=1e-5)
    dx = np.zeros((M, K), np.float32)
    orc.call("linear_bwd_dx", dx, dY, W, M, N, K)
    np.testing.assert_allclose(dx, dY64 @ W64, rtol=1e-6, atol=1e-5)
    dw0 = f32(r.standard_normal((N, K)))
    dw = dw0.copy()
    orc.call("linear_bwd_dw", dw, dY, X, M, N, K)
    np.testing.assert_allclose(dw, dw0 + dY64.T @ X64, rtol=1e-6, atol=1e-5)
    # in place dX (model.mojo:906): reads all of dY first
    if N == K:
        buf = dY.copy()
        orc.call("linear_bwd_dx", buf, buf, W, M, N, K)
        np.testing.assert_allclose(buf, dY64 @ W64, rtol=1e-6, atol=1e-5)


def test_rope_properties():
    r = np.random.default_rng(1)
    nt, H, hd = 40, 3, 64
    c, s = np.zeros((nt, hd // 2), np.float32), np.zeros((nt, hd // 2), np.float32)
    orc.call("precompute_rope", c, s, nt, hd, 10000.0)
    t = np.arange(nt)[:, None]
    freq = t / 10000.0 ** (2 * np.arange(hd // 2)[None, :] / hd)  # model.mojo:72-78
    np.testing.assert_array_equal(c, np.cos(freq).astype(np.float32))
    x = f32(r.standard_normal((nt, H, hd)))
    y, back = np.zeros_like(x), np.zeros_like(x)
    orc.call("rope_fwd", y, x, c, s, nt, H, hd)
    orc.call("rope_bwd", back, y, c, s, nt, H, hd)
    np.testing.assert_allclose(back, x, atol=1e-5)  # inverse rotation
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)
    # closed form of one pair
    x1, x2 = x[:, :, :hd // 2], x[:, :, hd // 2:]
    cc, ss = c[:, None, :], s[:, None, :]
    np.testing.assert_allclose(y[:, :, :hd // 2], x1 * cc + x2 * ss, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(y[:, :, hd // 2:], -x1 * ss + x2 * cc, rtol=1e-6, atol=1e-6)


def _torch_attn(q, k, v, window):
    B, T, H, hd = q.shape
    qt, kt, vt = (x.permute(0, 2, 1, 3) for x in (q, k, v))
    s = qt @ kt.transpose(-1, -2) / np.sqrt(hd)
    i = torch.arange(T)
    vis = i[None, :] <= i[:, None]
    if window > 0:
        vis &= i[None, :] >= i[:, None] - window
    s = s.masked_fill(~vis, float("-inf"))
    lse = torch.logsumexp(s, -1)
    o = torch.softmax(s, -1) @ vt
    return o.permute(0, 2, 1, 3), lse.permute(0, 2, 1)


@pytest.mark.parametrize("window", [0, 5, 16])
def test_attention_vs_torch_autograd(window):
    r = np.random.default_rng(window)
    B, T, H, hd = 2, 23, 2, 16
    q, k, v, do = (f32(r.standard_normal((B, T, H, hd))) for _ in range(4))
    n = B * T * H
    o, lse = np.zeros_like(q), np.zeros(n, np.float32)
    orc.call("flash_attn_fwd", o, lse, q, k, v, B, T, H, hd, window)
    qt, kt, vt = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
    ot, lt = _torch_attn(qt, kt, vt, window)
    np.testing.assert_allclose(o, ot.detach().numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lse, lt.detach().numpy().ravel(), rtol=1e-6, atol=1e-6)
    ot.backward(torch.tensor(do, dtype=torch.float64))
    d = np.zeros(n, np.float32)
    orc.call("flash_attn_bwd_precompute_d", d, o, do, B, T, H, hd)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(q), np.zeros_like(q)
    orc.call("flash_attn_bwd_dq", dq, q, k, v, do, lse, d, B, T, H, hd, window)
    orc.call("flash_attn_bwd_dkv", dk, dv, q, k, v, do, lse, d, B, T, H, hd, window)
    for a, g in ((dq, qt), (dk, kt), (dv, vt)):
        np.testing.assert_allclose(a, g.grad.numpy(), rtol=1e-4, atol=1e-5)


def test_cross_entropy_vs_torch():
    r = np.random.default_rng(2)
    nt, V = 19, 50
    z = f32(r.standard_normal((nt, V)) * 5)
    tg = r.integers(0, V, nt).astype(np.int64)
    tg[3] = -1
    loss = np.zeros(nt, np.float32)
    orc.call("cross_entropy_fwd", loss, z, tg, nt, V)
    ref = torch.nn.functional.cross_entropy(torch.tensor(z, dtype=torch.float64), torch.tensor(tg),
                                            reduction="none", ignore_index=-1).numpy()
    np.testing.assert_allclose(loss, ref, rtol=1e-6, atol=1e-6)
    g = np.zeros_like(z)
    orc.call("cross_entropy_softcap_bwd", g, z, tg, 15.0, nt, V, 0.25)
    sm = torch.softmax(torch.tensor(z, dtype=torch.float64), -1).numpy()
    oh = np.zeros_like(sm)
    oh[np.arange(nt), np.maximum(tg, 0)] = 1.0
    exp = (sm - oh) * 0.25
    exp[3] = 0.0  # ignored target row (ops.mojo:801-804)
    np.testing.assert_allclose(g, exp, rtol=1e-5, atol=1e-7)
    m = np.zeros(1, np.float32)
    orc.call("mean_reduce", m, loss, nt)
    assert abs(m[0] - loss.astype(np.float64).mean()) <= 1e-6


def test_softcap_and_relu2_vs_torch():
    r = np.random.default_rng(3)
    x = f32(r.standard_normal(1000) * 30)
    y = np.zeros_like(x)
    orc.call("softcap_fwd", y, x, 15.0, x.size)
    np.testing.assert_allclose(y, 15.0 * np.tanh(x.astype(np.float64) / 15.0), rtol=1e-6, atol=1e-6)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    (torch.relu(xt) ** 2).backward(torch.ones_like(xt))
    g = np.zeros_like(x)
    orc.call("relu_squared_bwd", g, np.ones_like(x), x, x.size)
    np.testing.assert_allclose(g, xt.grad.numpy(), rtol=1e-6)


def test_value_embedding_vs_autograd():
    r = np.random.default_rng(4)
    nt, H, hd, gc, C = 11, 3, 8, 32, 40
    xn = f32(r.standard_normal((nt, C)))
    w = f32(r.standard_normal((H, gc)) * 0.3)
    v0, ve, gv = (f32(r.standard_normal((nt, H, hd))) for _ in range(3))
    gate = np.zeros((nt, H), np.float32)
    orc.call("ve_gate_fwd", gate, xn, w, nt, H, gc, C)
    xt = torch.tensor(xn, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    vet = torch.tensor(ve, dtype=torch.float64, requires_grad=True)
    gt = 2 * torch.sigmoid(xt[:, :gc] @ wt.T)
    np.testing.assert_allclose(gate, gt.detach().numpy(), rtol=1e-6)
    out = torch.tensor(v0, dtype=torch.float64) + gt[:, :, None] * vet
    out.backward(torch.tensor(gv, dtype=torch.float64))
    v = v0.copy()
    orc.call("ve_apply_fwd", v, gate, ve, nt, H, hd)
    np.testing.assert_allclose(v, out.detach().numpy(), rtol=1e-5, atol=1e-6)
    gve, gg = np.zeros_like(ve), np.zeros((nt, H), np.float32)
    orc.call("ve_apply_bwd", gve, gg, gv, gate, ve, nt, H, hd)
    np.testing.assert_allclose(gve, vet.grad.numpy(), rtol=1e-5, atol=1e-6)
    gx, gw = np.zeros_like(xn), np.zeros_like(w)
    orc.call("ve_gate_bwd", gx, gw, gg, gate, xn, w, nt, H, gc, C)
    np.testing.assert_allclose(gx, xt.grad.numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(gw, wt.grad.numpy(), rtol=1e-5, atol=1e-6)


def test_residual_kernels():
    r = np.random.default_rng(5)
    a, b, g = (f32(r.standard_normal(100)) for _ in range(3))
    sa, sb = f32([1.5, 0.5]), f32([0.1, -2.0])
    out = np.zeros_like(a)
    orc.call("scaled_add_fwd", out, a, b, sa, sb, 1, 100)
    np.testing.assert_array_equal(out, f32(sa[1] * a) + f32(sb[1] * b))
    ga, gb = g.copy(), np.zeros_like(g)
    orc.call("scaled_add_bwd", ga, gb, ga, sa, sb, 0, 100)
    np.testing.assert_array_equal(ga, f32(sa[0] * g))
    np.testing.assert_array_equal(gb, f32(sb[0] * g))
    gs = f32([0.0, 1.0])
    orc.call("scalar_grad_reduce", gs, a, b, 1, 100)
    assert abs(gs[1] - (1.0 + (a.astype(np.float64) * b).sum())) <= 1e-5


def test_embedding_bwd_matches_token_order_sum():
    r = np.random.default_rng(6)
    n, V, D = 700, 30, 12
    p = 1.0 / np.arange(1, V + 1) ** 1.1
    idx = r.choice(V, n, p=p / p.sum()).astype(np.int64)
    # integer-valued data: every summation order is exact, so the chunked
    # order must equal the plain token-order scatter bit for bit
    dy = f32(r.integers(-50, 50, (n, D)))
    g0 = f32(r.integers(-50, 50, (V, D)))
    gw = g0.copy()
    orc.call("embedding_bwd", gw, dy, idx, n, D)
    ref = g0.astype(np.float64).copy()
    np.add.at(ref, idx, dy.astype(np.float64))
    np.testing.assert_array_equal(gw, ref.astype(np.float32))
    dyr = f32(r.standard_normal((n, D)))
    gw = np.zeros((V, D), np.float32)
    orc.call("embedding_bwd", gw, dyr, idx, n, D)
    ref = np.zeros((V, D))
    np.add.at(ref, idx, dyr.astype(np.float64))
    np.testing.assert_allclose(gw, ref, rtol=1e-5, atol=1e-5)


def test_adamw_vs_torch():
    r = np.random.default_rng(7)
    p0, g = f32(r.standard_normal(500)), f32(r.standard_normal(500) * 0.1)
    pt = torch.tensor(p0, dtype=torch.float64, requires_grad=True)
    opt = torch.optim.AdamW([pt], lr=0.01, betas=(0.8, 0.95), eps=1e-10, weight_decay=0.1)
    p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    for step in range(1, 4):
        pt.grad = torch.tensor(g * step, dtype=torch.float64)
        opt.step()
        bc1, bc2 = np.float32(1.0), np.float32(1.0)
        for _ in range(step):
            bc1, bc2 = np.float32(bc1 * np.float32(0.8)), np.float32(bc2 * np.float32(0.95))
        orc.call("adamw", p, f32(g * step), m, v, 0.01, 0.8, 0.95, 1e-10, 0.1, float(1 - bc1), float(1 - bc2), 500)
    np.testing.assert_allclose(p, pt.detach().numpy(), rtol=1e-5, atol=1e-6)


def _polar(grad, rows, cols):
    """Muon update direction X (params start at 0, lr 1, no decay)."""
    p, g, mb = np.zeros((rows, cols), np.float32), f32(grad).copy(), np.zeros((rows, cols), np.float32)
    orc.call("muon_step", p, g, mb, rows, cols, 1.0, 1.0, 0.0, 0.0)
    lr = np.sqrt(rows / cols) if rows > cols else 1.0
    return -p / lr


def test_muon_orthogonalizes_and_is_transpose_equivariant():
    r = np.random.default_rng(8)
    G = f32(r.standard_normal((96, 32)))
    X = _polar(G, 96, 32).astype(np.float64)
    sv = np.linalg.svd(X, compute_uv=False)
    assert sv.min() > 0.5 and sv.max() < 1.3, sv  # singular values pushed towards 1
    # same singular vectors as G (X is a polynomial in G G^T applied to G)
    U, S, Vt = np.linalg.svd(G.astype(np.float64), full_matrices=False)
    Xr = U.T @ X @ Vt.T
    assert np.abs(Xr - np.diag(np.diag(Xr))).max() < 1e-3
    # wide path on G^T gives the transpose of the tall path on G
    Xw = _polar(np.ascontiguousarray(G.T), 32, 96).astype(np.float64)
    np.testing.assert_allclose(Xw, X.T, rtol=1e-3, atol=1e-4)
    # Nesterov momentum: out = (1-mu) g + mu (mu buf + (1-mu) g)
    out, buf = np.zeros(10, np.float32), f32(np.arange(10))
    gg = f32(np.ones(10))
    orc.call("nesterov_momentum", out, gg, buf, 0.9, 10)
    np.testing.assert_allclose(buf, 0.9 * np.arange(10) + 0.1, rtol=1e-6)
    np.testing.assert_allclose(out, 0.1 + 0.9 * buf, rtol=1e-6)


def _prng_states(seed, n):
    with np.errstate(over="ignore"):
        i = np.arange(n, dtype=np.uint64)
        st = np.uint64(seed) + i * np.uint64(6364136223846793005) + np.uint64(1442695040888963407)
        st ^= st >> np.uint64(12)
        st ^= st << np.uint64(25)
        st ^= st >> np.uint64(27)
    return st


def test_init_prng_independent_restatement():
    n, seed = 5000, 45
    st = _prng_states(seed, n)
    u = (st & np.uint64(0xFFFFFF)).astype(np.float32) / np.float32(16777216.0)
    lo, hi = np.float32(-0.0765), np.float32(0.0765)
    ref = lo + (u * np.float32(hi - lo)).astype(np.float32)
    out = np.zeros(n, np.float32)
    orc.call("fill_uniform", out, seed, float(lo), float(hi), n)
    np.testing.assert_array_equal(out, ref.astype(np.float32))  # bit-exact
    with np.errstate(over="ignore"):
        st2 = st * np.uint64(6364136223846793005) + np.uint64(1442695040888963407)
        st2 ^= st2 >> np.uint64(12)
        st2 ^= st2 << np.uint64(25)
        st2 ^= st2 >> np.uint64(27)
    u1 = (st & np.uint64(0xFFFFFF)).astype(np.float64) / 16777216.0 + 1e-10
    u2 = (st2 & np.uint64(0xFFFFFF)).astype(np.float64) / 16777216.0
    z = np.sqrt(-2 * np.log(u1)) * np.cos(2 * np.pi * u2)
    orc.call("fill_normal", out, seed, 1.0, n)
    np.testing.assert_allclose(out, z, rtol=1e-5, atol=2e-6)


# ---------------- whole model ----------------
CFG1 = dict(sequence_len=64, vocab_size=512, n_layer=2, n_head=2, n_kv_head=2, n_embd=128, head_dim=64, kv_dim=128)


def _batch(seed, B, T, V):
    t = np.random.default_rng(seed).integers(0, V, (B, T + 1)).astype(np.int64)
    return np.ascontiguousarray(t[:, :-1]).ravel(), np.ascontiguousarray(t[:, 1:]).ravel()


def test_model_behaviour_config1():
    m = orc.Model(CFG1, 2, 64, 0)
    m.init_weights(0)
    x, y = _batch(0, 2, 64, 512)
    m.zero_grads()
    loss = m.forward(x, y)
    # lm_head ~ N(0, 0.001): near-uniform logits (test_forward.mojo:114-120 bounds)
    assert abs(loss - np.log(512)) < 0.01
    m.backward(x, y)
    g = m.grads()
    names = {n: (o, s) for n, o, s in m.tensors()}
    for nm in ("h0.c_q", "h0.c_k", "h0.c_v", "h0.c_fc", "h1.c_q"):
        o, s = names[nm]
        assert np.all(g[o:o + s] == 0.0), nm  # c_proj / mlp_proj start at zero
    for nm in ("lm_head", "wte", "h1.c_proj", "h1.mlp_proj"):
        o, s = names[nm]
        assert np.any(g[o:o + s] != 0.0), nm  # test_backward.mojo:98-129
    losses = [m.train_step(x, y, 0.0) for _ in range(6)]
    assert losses[-1] < losses[0] and np.all(np.isfinite(losses))


def test_model_lm_head_gradient_finite_difference():
    """At init the logits are tiny (|z| << 15), so the reference's CE+softcap
    backward (no tanh' factor, Q4) equals the true gradient of the summed loss
    (Q5) to ~1e-6: central differences of sum(loss) pin the lm_head gradient."""
    m = orc.Model(CFG1, 2, 64, 0)
    m.init_weights(3)
    x, y = _batch(1, 2, 64, 512)
    m.zero_grads()
    m.forward(x, y)
    m.backward(x, y)
    names = {n: (o, s) for n, o, s in m.tensors()}
    o, s = names["lm_head"]
    g = m.grads()[o:o + s].copy()
    p = m.params()
    r = np.random.default_rng(0)
    for j in r.choice(s, 6, replace=False):
        old = p[o + j]
        h = 1e-2
        p[o + j] = old + h
        lp = m.forward(x, y) * 128
        p[o + j] = old - h
        lm = m.forward(x, y) * 128
        p[o + j] = old
        fd = (lp - lm) / (2 * h)
        assert abs(fd - g[j]) <= 2e-3 * max(1.0, abs(g[j])), (j, fd, g[j])


def test_model_released_cleanly_at_interpreter_exit():
    """An oracle Model still alive when the interpreter exits is destroyed
    without an 'Exception ignored' report (module globals may already be gone)."""
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = ("from oracle import oracle as orc\n"
            "m = orc.Model(dict(sequence_len=64, vocab_size=512, n_layer=2, n_head=2, n_kv_head=2, n_embd=128,"
            " head_dim=64, kv_dim=128), 2, 64, 0)\n")
    r = subprocess.run([sys.executable, "-c", code], cwd=root, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "Exception ignored" not in r.stderr, r.stderr
