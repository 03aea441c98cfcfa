"""Pins the oracle's whole-step composites (orc_model_forward, _backward and
_optimizer_step) against restatements written independently of it, from the
reference's own source:

* an fp64 torch-autograd GPT following model.mojo's forward
  (model.mojo:576-772).  Where the reference backward (model.mojo:819-1037)
  is not the true gradient, the deviation is expressed as a small autograd
  rule of its own:
    Q4  softcap backward skipped (ops.mojo:854-858)       -> straight-through
    Q5  backward of the summed loss (train.mojo:238)      -> sum().backward()
    Q6  q/k head-norm backward skipped (model.mojo:937)   -> straight-through
    Q7  MLP-norm backward on the layer's saved pre-attention x with the MLP
        rms (model.mojo:892-896)                          -> _MlpNorm
    Q8  resid_lambdas gradient = sum g * post-scaled x (model.mojo:1010-1014)
    Q9  grad_x0 assigned and never consumed (ops.mojo:1189-1190) -> _ScaledAdd
    Q10 embedding-norm backward skipped (model.mojo:1028-1031) -> straight-through
* a numpy fp64 restatement of the optimizer wiring: the AdamW groups
  (train.mojo:166-186, optimizer.mojo:27-57, 103-127) and Muon
  (train.mojo:188-196, 264-281; optimizer.mojo:132-342), fed the same
  gradients as the oracle for two steps;
* the closed form of Polar Express: with X = U S V^T every iteration maps each
  singular value s to a s + b s^3 + c s^5 (the products X^T X, b A + c A A and
  a X + X B keep U and V), so after Frobenius normalisation the five
  iterations of config.mojo:93-112 fix the singular values exactly.  A wrong
  coefficient order, a transposed product or a dropped term fails it.

CPU only."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc

D = torch.float64
EPS = 1e-5        # ops.mojo:98-104
SOFTCAP = 15.0    # config.mojo:86
GATE_CH = 32      # config.mojo:64
# config.mojo:93-112, (a, b, c) per iteration
POLAR = [(8.156554524902461, -22.48329292557795, 15.878769915207462),
         (4.042929935166739, -2.808917465908714, 0.5000178451051316),
         (3.8916678022926607, -2.772484153217685, 0.5060648178503393),
         (3.285753657755655, -2.3681294933425376, 0.46449024233003106),
         (2.3465413258596377, -1.7097828382687081, 0.42323551169305323)]

CFG1 = dict(sequence_len=64, vocab_size=512, n_layer=2, n_head=2, n_kv_head=2, n_embd=128, head_dim=64, kv_dim=128)
# four layers: value embeddings on layers 1 and 3, windows [32, 32, 32, 64]
CFG4L = dict(sequence_len=64, vocab_size=256, n_layer=4, n_head=2, n_kv_head=2, n_embd=128, head_dim=64,
             kv_dim=128)


def _has_ve(cfg, i):  # config.mojo:45-47
    return i % 2 == (cfg["n_layer"] - 1) % 2


def _window(cfg, i):  # config.mojo:49-55
    T = cfg["sequence_len"]
    if i == cfg["n_layer"] - 1:
        return T
    return T // 2 if i % 4 < 3 else T


# ---------------- fp64 autograd model ----------------
def _rms(x):
    return torch.sqrt((x * x).mean(-1, keepdim=True) + EPS)


def _straight_through(x, y):
    """Value y, gradient passed to x unchanged."""
    return x + (y - x).detach()


class _MlpNorm(torch.autograd.Function):
    """Q7: value x_mid / rms(x_mid); backward applies the rmsnorm gradient
    formula (ops.mojo:1080-1085) to the saved pre-attention x with rms(x_mid)."""

    @staticmethod
    def forward(ctx, x_mid, x_saved):
        r = _rms(x_mid)
        ctx.save_for_backward(x_saved, r)
        return x_mid / r

    @staticmethod
    def backward(ctx, g):
        xs, r = ctx.saved_tensors
        C = xs.shape[-1]
        dot = (g * xs).sum(-1, keepdim=True)
        return (g - xs * dot / (C * r * r)) / r, None


class _ScaledAdd(torch.autograd.Function):
    """x = ra[i] x_prev + xa[i] x0 with the reference's backward: the x_prev
    gradient ra[i] g, ra's gradient sum(g * x) on the OUTPUT x (Q8), xa's
    sum(g * x0), and no gradient into x0 (Q9)."""

    @staticmethod
    def forward(ctx, x_prev, x0, ra, xa, i):
        out = ra[i] * x_prev + xa[i] * x0
        ctx.save_for_backward(out, x0, ra)
        ctx.i = i
        return out

    @staticmethod
    def backward(ctx, g):
        out, x0, ra = ctx.saved_tensors
        i = ctx.i
        g_ra = torch.zeros_like(ra)
        g_xa = torch.zeros_like(ra)
        g_ra[i] = (g * out).sum()
        g_xa[i] = (g * x0).sum()
        return ra[i] * g, None, g_ra, g_xa, None


def _rope_tables(rows, hd):
    """model.mojo:57-81: cos / sin(t / 10000^(2d/hd)) in f64, stored as f32."""
    t = np.arange(rows, dtype=np.float64)[:, None]
    d = np.arange(hd // 2, dtype=np.float64)[None, :]
    f = t / (10000.0 ** (2.0 * d / hd))
    return (torch.tensor(np.cos(f).astype(np.float32), dtype=D), torch.tensor(np.sin(f).astype(np.float32), dtype=D))


def _rope(x, cos, sin):
    """ops.mojo:209-238 on [BT, H, hd]: halves (x1, x2) -> (x1 c + x2 s, -x1 s + x2 c)."""
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    c, s = cos[:, None, :], sin[:, None, :]
    return torch.cat([x1 * c + x2 * s, -x1 * s + x2 * c], -1)


# ---- bf16 operand storage, emulated in fp64 ----
# A bf16-mode step stores every matrix-product operand as bf16 in both passes:
# a product's inputs and the gradient that reaches its output (dY), plus the
# attention probabilities P (for P V) and dS (for dQ, dK).  _round_both rounds
# a value and the gradient that flows back through it; _round_grad only the
# gradient; _round_value only the value.  The distance of this model's
# gradients from the exact fp64 ones measures how far bf16 rounding alone
# moves each gradient (large where a gradient is a small difference of large
# terms).
def _bf(x):
    return x.to(torch.bfloat16).to(x.dtype)


class _RoundBoth(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        return _bf(x)

    @staticmethod
    def backward(ctx, g):
        return _bf(g)


class _RoundGrad(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        return x.clone()

    @staticmethod
    def backward(ctx, g):
        return _bf(g)


class _RoundValue(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        return _bf(x)

    @staticmethod
    def backward(ctx, g):
        return g


def _mm(a, b, bf16):
    if not bf16:
        return a @ b
    return _RoundGrad.apply(_RoundBoth.apply(a) @ _RoundBoth.apply(b))


def _attention(q, k, v, B, T, ws, bf16=False):
    """Key kp visible from qp iff kp <= qp and (ws <= 0 or kp >= qp - ws),
    scores scaled by 1/sqrt(hd) (ops.mojo:244-323).  q, k, v: [B*T, H, hd]."""
    H, hd = q.shape[1], q.shape[2]
    if bf16:
        q, k, v = _RoundBoth.apply(q), _RoundBoth.apply(k), _RoundBoth.apply(v)
    qt, kt, vt = (x.reshape(B, T, H, hd).permute(0, 2, 1, 3) for x in (q, k, v))
    s = qt @ kt.transpose(-1, -2) / np.sqrt(hd)
    if bf16:
        s = _RoundGrad.apply(s)  # dS
    i = torch.arange(T)
    vis = i[None, :] <= i[:, None]
    if ws > 0:
        vis = vis & (i[None, :] >= i[:, None] - ws)
    s = s.masked_fill(~vis, float("-inf"))
    p = torch.softmax(s, -1)
    o = (_RoundValue.apply(p) if bf16 else p) @ vt
    return o.permute(0, 2, 1, 3).reshape(B * T, H, hd)


def _torch_step(cfg, W, x_ids, y_ids, B, T, rope_period, bf16=False):
    """Forward of model.mojo:576-772 in fp64; returns (mean loss, per-token
    loss, {name: gradient}) with the reference backward's rules.  bf16: every
    product operand rounded to bf16 as above (the rest stays fp64)."""
    C, V, L, H, hd = cfg["n_embd"], cfg["vocab_size"], cfg["n_layer"], cfg["n_head"], cfg["head_dim"]
    BT = B * T
    P = {n: torch.tensor(a, dtype=D, requires_grad=True) for n, a in W.items()}
    pos = np.arange(BT) % rope_period if rope_period > 0 else np.arange(BT)
    cos_t, sin_t = _rope_tables(int(pos.max()) + 1, hd)
    cos, sin = cos_t[pos], sin_t[pos]
    ids = torch.tensor(x_ids)
    e = P["wte"][ids]
    x0 = _straight_through(e, e / _rms(e))                         # Q10
    x = x0
    for i in range(L):
        p = f"h{i}."
        x = _ScaledAdd.apply(x, x0.detach(), P["resid_lambdas"], P["x0_lambdas"], i)
        x_saved = x
        xn = x / _rms(x)
        q = _mm(xn, P[p + "c_q"].T, bf16).reshape(BT, H, hd)
        k = _mm(xn, P[p + "c_k"].T, bf16).reshape(BT, H, hd)
        v = _mm(xn, P[p + "c_v"].T, bf16).reshape(BT, H, hd)
        if _has_ve(cfg, i):
            ve = P[p + "value_embeds"][ids].reshape(BT, H, hd)
            gate = 2.0 * torch.sigmoid(xn[:, :GATE_CH] @ P[p + "ve_gate"].T)   # [BT, H]
            v = v + gate[:, :, None] * ve
        q, k = _rope(q, cos, sin), _rope(k, cos, sin)
        q = _straight_through(q, q / _rms(q))                       # Q6
        k = _straight_through(k, k / _rms(k))
        a = _attention(q, k, v, B, T, _window(cfg, i), bf16).reshape(BT, C)
        x = x + _mm(a, P[p + "c_proj"].T, bf16)
        xn2 = _MlpNorm.apply(x, x_saved)                            # Q7
        act = torch.relu(_mm(xn2, P[p + "c_fc"].T, bf16)) ** 2
        x = x + _mm(act, P[p + "mlp_proj"].T, bf16)
    xf = x / _rms(x)
    z = _mm(xf, P["lm_head"].T, bf16)
    zc = _straight_through(z, SOFTCAP * torch.tanh(z / SOFTCAP))    # Q4
    tok = torch.logsumexp(zc, -1) - zc[torch.arange(BT), torch.tensor(y_ids)]
    tok.sum().backward()                                            # Q5
    return float(tok.detach().mean()), tok.detach().numpy(), {n: t.grad.numpy() for n, t in P.items()}


def _random_weights(cfg, om, seed):
    """Every tensor random and non-zero (at init c_proj, mlp_proj and the
    gates are zero, which would leave most of the backward untested).  The
    oracle's init also fills its RoPE table, so it runs first."""
    om.init_weights(seed)
    r = np.random.default_rng(seed)
    C = cfg["n_embd"]
    W = {}
    for n, o, s in om.tensors():
        if n == "wte":
            a = r.standard_normal(s)
        elif n == "lm_head":
            a = r.standard_normal(s) * 0.3  # logits of a few units: tanh' well below 1
        elif n == "resid_lambdas":
            a = 1.0 + 0.1 * r.standard_normal(s)
        elif n == "x0_lambdas":
            a = 0.1 + 0.05 * r.standard_normal(s)
        elif n.endswith("ve_gate"):
            a = r.standard_normal(s) * 0.3
        elif n.endswith("value_embeds"):
            a = r.standard_normal(s) * 0.5
        else:
            a = r.standard_normal(s) * (0.8 / np.sqrt(C))
        W[n] = a.astype(np.float32)
    return W


def _shapes(cfg):
    C, V, L, H = cfg["n_embd"], cfg["vocab_size"], cfg["n_layer"], cfg["n_head"]
    kv = cfg["kv_dim"]
    sh = {"wte": (V, C), "lm_head": (V, C), "resid_lambdas": (L,), "x0_lambdas": (L,)}
    for i in range(L):
        p = f"h{i}."
        sh.update({p + "c_q": (C, C), p + "c_k": (kv, C), p + "c_v": (kv, C), p + "c_proj": (C, C),
                   p + "c_fc": (4 * C, C), p + "mlp_proj": (C, 4 * C)})
        if _has_ve(cfg, i):
            sh.update({p + "value_embeds": (V, kv), p + "ve_gate": (H, GATE_CH)})
    return sh


def _rel(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    nb = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / nb) if nb > 0 else float(np.linalg.norm(a - b))


@pytest.mark.parametrize("cfg,B,T,period,seed", [(CFG1, 2, 64, 0, 11), (CFG4L, 2, 64, 64, 12)])
def test_forward_backward_vs_fp64_autograd(cfg, B, T, period, seed):
    """Loss, per-token loss and every parameter gradient of orc_model_forward /
    orc_model_backward against the fp64 autograd restatement, on random
    non-zero weights (config 1 with flat-token RoPE rows; a four-layer model
    with two value-embedding layers, short windows and per-sequence RoPE)."""
    om = orc.Model(cfg, B, T, period)
    W = _random_weights(cfg, om, seed)
    sh = _shapes(cfg)
    p = om.params()
    for n, o, s in om.tensors():
        p[o:o + s] = W[n]
    r = np.random.default_rng(seed + 100)
    toks = r.integers(0, cfg["vocab_size"], (B, T + 1)).astype(np.int64)
    x, y = np.ascontiguousarray(toks[:, :-1]).ravel(), np.ascontiguousarray(toks[:, 1:]).ravel()
    om.zero_grads()
    loss_o = om.forward(x, y)
    tok_o = om.token_loss().copy()
    om.backward(x, y, 1.0)
    g_o = om.grads()
    loss_t, tok_t, g_t = _torch_step(cfg, {n: W[n].reshape(sh[n]) for n in W}, x, y, B, T, period)
    assert abs(loss_o - loss_t) <= 2e-6 * abs(loss_t), (loss_o, loss_t)
    assert _rel(tok_o, tok_t) <= 2e-6
    for n, o, s in om.tensors():
        gt = g_t[n].ravel()
        assert np.linalg.norm(gt) > 0, n  # every gradient is exercised
        assert _rel(g_o[o:o + s], gt) <= 1e-5, (n, _rel(g_o[o:o + s], gt))


def test_quirk_rules_change_the_gradient():
    """Each quirk rule of the restatement matters: with the true gradient in
    its place the comparison above would fail, so none of them is vacuous."""
    cfg, B, T = CFG4L, 2, 64
    om = orc.Model(cfg, B, T, 64)
    W = _random_weights(cfg, om, 12)
    sh = _shapes(cfg)
    Wd = {n: W[n].reshape(sh[n]) for n in W}
    r = np.random.default_rng(112)
    toks = r.integers(0, cfg["vocab_size"], (B, T + 1)).astype(np.int64)
    x, y = np.ascontiguousarray(toks[:, :-1]).ravel(), np.ascontiguousarray(toks[:, 1:]).ravel()
    _, _, g_ref = _torch_step(cfg, Wd, x, y, B, T, 64)
    global _MlpNorm, _straight_through
    saved = (_MlpNorm, _straight_through)
    try:
        # Q7 with the true rmsnorm gradient of x_mid
        class _TrueNorm(torch.autograd.Function):
            @staticmethod
            def forward(ctx, xm, xs):
                ctx.save_for_backward(xm)
                return xm / _rms(xm)

            @staticmethod
            def backward(ctx, g):
                (xm,) = ctx.saved_tensors
                r_ = _rms(xm)
                return (g - xm * (g * xm).sum(-1, keepdim=True) / (xm.shape[-1] * r_ * r_)) / r_, None
        _MlpNorm = _TrueNorm
        _, _, g = _torch_step(cfg, Wd, x, y, B, T, 64)
        assert _rel(g["h0.c_q"], g_ref["h0.c_q"]) > 1e-3
        _MlpNorm = saved[0]
        # Q4 / Q6 / Q10 with true gradients
        _straight_through = lambda a, b: b  # noqa: E731
        _, _, g = _torch_step(cfg, Wd, x, y, B, T, 64)
        assert _rel(g["lm_head"], g_ref["lm_head"]) > 1e-4
        assert _rel(g["h0.c_q"], g_ref["h0.c_q"]) > 1e-3
        assert _rel(g["wte"], g_ref["wte"]) > 1e-3
    finally:
        _MlpNorm, _straight_through = saved


# ---------------- optimizer wiring ----------------
def _f32(v):
    return float(np.float32(v))


def _lr_multiplier(progress):  # train.mojo:25-33 with config.mojo:81-83
    warmup, warmdown, final = 0.0, 0.5, 0.0
    if progress < warmup:
        return progress / warmup if warmup > 0 else 1.0
    if progress < 1.0 - warmdown:
        return 1.0
    cd = (1.0 - progress) / warmdown
    return cd + (1.0 - cd) * final


def _polar_express(G, rows, cols):
    """optimizer.mojo:292-337 in fp64: tall (rows >= cols) A = X^T X, X' = a X + X B;
    wide A = X X^T, X' = a X + B X; B = b A + c A A."""
    X = G.astype(np.float64)
    for a, b, c in POLAR:
        if rows >= cols:
            A = X.T @ X
            X = a * X + X @ (b * A + c * (A @ A))
        else:
            A = X @ X.T
            X = a * X + (b * A + c * (A @ A)) @ X
    return X


class _NumpyOptimizer:
    """train.mojo:166-196 groups, stepped as train.mojo:246-281."""

    def __init__(self, cfg, tensors):
        self.cfg = cfg
        self.t = {n: (o, s) for n, o, s in tensors}
        self.m = {n: np.zeros(s) for n, _, s in tensors}
        self.v = {n: np.zeros(s) for n, _, s in tensors}
        self.buf = {n: np.zeros(s) for n, _, s in tensors}
        self.step = 0
        # per Muon matrix: entries whose cautious-decay decision sign(X p) is
        # within rounding of 0 (fp32 and fp64 may take either branch there),
        # and the decay term lr wd p that separates the two branches
        self.ambiguous, self.decay = {}, {}

    def __call__(self, params, grads, progress):
        cfg = self.cfg
        C, L, kv = cfg["n_embd"], cfg["n_layer"], cfg["kv_dim"]
        lrm = _lr_multiplier(min(progress, 1.0))
        s = (C / 768.0) ** -0.5
        self.step += 1
        out = {n: params[o:o + sz].astype(np.float64) for n, (o, sz) in self.t.items()}
        g = {n: grads[o:o + sz].astype(np.float64) for n, (o, sz) in self.t.items()}
        adam = [("lm_head", 0.004 * s, 0.8), ("wte", 0.6 * s, 0.8), ("resid_lambdas", 0.5 * 0.01, 0.8),
                ("x0_lambdas", 0.5, 0.96)]
        for i in range(L):
            if _has_ve(cfg, i):
                adam += [(f"h{i}.value_embeds", 0.6 * s, 0.8), (f"h{i}.ve_gate", 0.04, 0.8)]
        for n, lr_g, b1 in adam:
            lr = _f32(lr_g * lrm)
            bc1 = bc2 = np.float32(1.0)
            for _ in range(self.step):  # optimizer.mojo:114-118
                bc1 = np.float32(bc1 * np.float32(b1))
                bc2 = np.float32(bc2 * np.float32(0.95))
            b1f, b2f = _f32(b1), _f32(0.95)
            self.m[n] = b1f * self.m[n] + (1 - b1f) * g[n]
            self.v[n] = b2f * self.v[n] + (1 - b2f) * g[n] ** 2
            out[n] = out[n] - lr * (self.m[n] / float(1 - bc1)) / (np.sqrt(self.v[n] / float(1 - bc2)) + _f32(1e-10))
        frac = min(self.step / 300.0, 1.0)
        mu = _f32((1.0 - frac) * 0.85 + frac * 0.95)
        wd = _f32(0.2 * (1.0 - min(progress, 1.0)))
        for i in range(L):
            for nm, rows, cols in (("c_q", C, C), ("c_k", kv, C), ("c_v", kv, C), ("c_proj", C, C),
                                   ("c_fc", 4 * C, C), ("mlp_proj", C, 4 * C)):
                n = f"h{i}.{nm}"
                aspect = rows / cols
                lr = _f32(0.04 * lrm * (np.sqrt(aspect) if aspect > 1.0 else 1.0))
                self.buf[n] = mu * self.buf[n] + (1 - mu) * g[n]
                X = (1 - mu) * g[n] + mu * self.buf[n]
                X = X / (np.linalg.norm(X) * 1.02 + 1e-6)
                X = _polar_express(X.reshape(rows, cols), rows, cols).ravel()
                p = out[n]
                self.ambiguous[n] = np.abs(X) <= 1e-4 * np.sqrt(np.mean(X * X))
                self.decay[n] = lr * wd * np.abs(p)
                out[n] = p - lr * (X + wd * p * (X * p >= 0))
        return out


@pytest.mark.parametrize("cfg", [CFG1, CFG4L])
def test_optimizer_step_vs_numpy_restatement(cfg):
    """Two optimizer steps of orc_model_optimizer_step (progress 0.0 then 0.8,
    i.e. lr multiplier 1 then 0.4 and weight decay 0.2 then 0.04) against the
    numpy restatement, from the same weights and the same gradients."""
    B, T = 1, 64
    om = orc.Model(cfg, B, T, 64)
    W = _random_weights(cfg, om, 21)
    p = om.params()
    for n, o, s in om.tensors():
        p[o:o + s] = W[n]
    opt = _NumpyOptimizer(cfg, om.tensors())
    r = np.random.default_rng(22)
    for progress in (0.0, 0.8):
        gr = om.grads()
        for n, o, s in om.tensors():
            gr[o:o + s] = (r.standard_normal(s) * r.choice([1e-3, 1e-1, 3.0])).astype(np.float32)
        pre = om.params().copy()
        want = opt(pre, gr.copy(), progress)
        om.optimizer_step(progress)
        got = om.params()
        for n, o, s in om.tensors():
            upd_o, upd_n = got[o:o + s].astype(np.float64) - pre[o:o + s], want[n] - pre[o:o + s]
            d = np.abs(upd_o - upd_n)
            # the fp32 weights quantise the oracle's update by half a spacing of the new weight
            quant = 0.5 * np.spacing(np.abs(got[o:o + s]))
            amb = opt.ambiguous.get(n, np.zeros(s, bool))
            if amb.any():  # either branch of the cautious decay, nothing else
                assert np.all(d[amb] <= opt.decay[n][amb] * 1.001 + 1e-5 * np.abs(upd_n[amb]) + quant[amb]), n
            ok = ~amb
            err = np.linalg.norm(d[ok]) - np.linalg.norm(quant[ok])
            assert err <= 2e-5 * np.linalg.norm(upd_n[ok]), (progress, n, err / np.linalg.norm(upd_n[ok]))


@pytest.mark.parametrize("rows,cols", [(96, 32), (32, 96), (64, 64)])
def test_polar_express_singular_values_closed_form(rows, cols):
    """orc_muon_step's direction X: its singular values equal the five
    Polar Express polynomials composed on s_i / (||G||_F 1.02 + 1e-6), and X
    keeps G's singular vectors."""
    r = np.random.default_rng(rows * 7 + cols)
    k = min(rows, cols)
    U, _ = np.linalg.qr(r.standard_normal((rows, k)))
    V, _ = np.linalg.qr(r.standard_normal((cols, k)))
    s = np.linspace(0.05, 1.0, k)[::-1]
    G = np.ascontiguousarray((U * s) @ V.T, dtype=np.float32)
    p, g, mb = np.zeros((rows, cols), np.float32), G.copy(), np.zeros((rows, cols), np.float32)
    orc.call("muon_step", p, g, mb, rows, cols, 1.0, 1.0, 0.0, 0.0)  # momentum 0: X = G; lr 1; wd 0
    lr = np.sqrt(rows / cols) if rows > cols else 1.0
    X = -p.astype(np.float64) / lr
    Gd = G.astype(np.float64)
    s0 = np.linalg.svd(Gd, compute_uv=False) / (np.linalg.norm(Gd) * 1.02 + 1e-6)
    want = s0.copy()
    for a, b, c in POLAR:
        want = a * want + b * want ** 3 + c * want ** 5
    got = np.linalg.svd(X, compute_uv=False)
    np.testing.assert_allclose(np.sort(got), np.sort(want), rtol=0, atol=2e-5)
    # the same from the fp64 product restatement (pins _polar_express as well)
    Xn = _polar_express(Gd / (np.linalg.norm(Gd) * 1.02 + 1e-6), rows, cols)
    np.testing.assert_allclose(np.sort(np.linalg.svd(Xn, compute_uv=False)), np.sort(want), rtol=0, atol=1e-9)
    # a reversed coefficient order moves the singular values well past the bound
    bad = s0.copy()
    for a, b, c in POLAR[::-1]:
        bad = a * bad + b * bad ** 3 + c * bad ** 5
    assert np.abs(np.sort(bad) - np.sort(want)).max() > 1e-2
