"""Whole training step on the GPU (ar_gpt_* through the C ABI) against the
CPU oracle: loss, every parameter gradient and the post-step weights, at
BASELINE config 1 (fp32 and bf16) and on a wider model with head_dim 128 and
sliding windows.  Gradients are captured before the optimizer step because
Muon clobbers them, as the reference does (optimizer.mojo:317-332)."""
import numpy as np
import pytest

from conftest import TOL_BF16, TOL_FP32, rel_err

pytestmark = pytest.mark.gpu

CONFIG1 = dict(sequence_len=64, vocab_size=512, n_layer=2, n_head=2, n_kv_head=2, n_embd=128, head_dim=64,
               kv_dim=128)
# Whole-model gradients chain ~40 fp32 GEMMs / reductions whose summation
# order legitimately differs from the oracle's double accumulation.
GRAD_FP32 = 3e-4
# Muon update error: the Polar Express polynomials multiply small singular
# values by prod(a_i) ~ 990 over five iterations, so fp32 operand rounding
# (6e-8) reaches a few 1e-4 of the update; bf16 operands a few 1e-2.
UPD_FP32 = 5e-4
UPD_BF16 = 6e-2   # Muon update, bf16 operands
WIDE = dict(sequence_len=256, vocab_size=1024, n_layer=4, n_head=2, n_kv_head=2, n_embd=256, head_dim=128,
            kv_dim=256)


def _tokens(seed, B, T, V):
    r = np.random.default_rng(seed)
    stream = r.integers(0, V, (B, T + 1)).astype(np.int64)
    return np.ascontiguousarray(stream[:, :-1]).ravel(), np.ascontiguousarray(stream[:, 1:]).ravel()


def _by_name(flat, tensors):
    return {n: np.array(flat[o:o + s], copy=True) for n, o, s in tensors}


def _copy_into(dst_flat, dst_tensors, src_flat, src_tensors):
    src = {n: (o, s) for n, o, s in src_tensors}
    for n, o, s in dst_tensors:
        so, ss = src[n]
        dst_flat[o:o + s] = src_flat[so:so + ss]


def _run(cfg, B, T, precision, rope_period, seed0, steps, tok_seed=0):
    """Each stage is compared on identical inputs: forward/backward from the
    same weights, then the optimizer from the same gradients (the GPU's are
    copied into the oracle), then weights are re-synchronised.  AdamW's first
    steps divide g by |g| and Muon normalises, so without this every ulp of
    gradient noise in a near-zero entry would show up as a weight mismatch."""
    import torch
    from autoresearch_amd.model import GPT, GPTConfig
    from oracle import oracle as orc
    import gpu_util as gu

    om = orc.Model(cfg, B, T, rope_period)
    om.init_weights(seed0)
    gm = GPT(GPTConfig(**cfg), B, T, precision=precision, rope_period=rope_period)
    gm.init_weights(seed0)
    ot, gt = om.tensors(), gm.tensors()
    assert [n for n, _, _ in ot] == [n for n, _, _ in gt]
    init_o, init_g = _by_name(om.params(), ot), _by_name(gu.host(gm.params()), gt)
    results = []
    for step in range(steps):
        # forward / backward start from identical weights
        _copy_into(om.params(), ot, gu.host(gm.params()), gt)
        x, y = _tokens(tok_seed + step, B, T, cfg["vocab_size"])
        xd, yd = gu.dev(x), gu.dev(y)
        om.zero_grads()
        lo = om.forward(x, y)
        om.backward(x, y, 1.0)
        gm.zero_grads()
        lg = gm.forward(xd, yd)
        gm.backward(xd, yd, 1.0)
        gflat = gu.host(gm.grads())
        go, gg = _by_name(om.grads().copy(), ot), _by_name(gflat, gt)
        l1 = om.scalar_grad_l1()
        tl_o, tl_g = om.token_loss().copy(), gu.host(gm.token_loss())
        # optimizer from identical gradients (and identical pre-step weights)
        _copy_into(om.grads(), ot, gflat, gt)
        pre = _by_name(gu.host(gm.params()), gt)
        om.optimizer_step(0.0)
        gm.optimizer_step(0.0)
        po, pg = _by_name(om.params().copy(), ot), _by_name(gu.host(gm.params()), gt)
        results.append(dict(loss=(lo, lg), tok=(tl_o, tl_g), grads=(go, gg), params=(po, pg), l1=l1, pre=pre))
    gm.close()
    return init_o, init_g, results


def _check(init_o, init_g, results, tol, grad_tol, upd_tol):
    """tol: loss / per-token loss / weights; grad_tol: every gradient;
    upd_tol: relative error allowed on the optimizer's update w_new - w_old.
    Muon's five Polar Express iterations amplify operand rounding (fp32 ~1e-4,
    bf16 operands ~5e-2 of the update); a weight's error is lr x that, so
    ||w_gpu - w_orc|| <= tol*||w_orc|| + upd_tol*||w_orc - w_old||."""
    # init is bit-exact for the uniform tensors, within fp32 for the normal ones
    for n in init_o:
        assert rel_err(init_g[n], init_o[n]) <= TOL_FP32, n
    for s, r in enumerate(results):
        lo, lg = r["loss"]
        assert abs(lg - lo) <= tol * abs(lo), (s, lo, lg)
        assert rel_err(r["tok"][1], r["tok"][0]) <= tol
        go, gg = r["grads"]
        # resid_lambdas / x0_lambdas gradients are sums of B*T*C products that
        # cancel to ~1e-3 of their L1 mass at init; fp32 noise in their inputs
        # is then amplified, so they are bounded by the summation error scale:
        # |diff| <= tol * sum_i |g_i x_i| (per layer).
        for n, l1 in (("resid_lambdas", r["l1"][0]), ("x0_lambdas", r["l1"][1])):
            assert np.all(np.abs(gg[n] - go[n]) <= grad_tol * l1), (s, n, gg[n], go[n], l1)
        for n in go:
            if n in ("resid_lambdas", "x0_lambdas"):
                continue
            if np.linalg.norm(go[n]) == 0.0:
                assert np.linalg.norm(gg[n]) == 0.0, (s, n)  # step 1: proj weights are zero
                continue
            assert rel_err(gg[n], go[n]) <= grad_tol, (s, n, rel_err(gg[n], go[n]))
        po, pg = r["params"]
        for n in po:
            w_old = r["pre"][n].astype(np.float64)
            bound = tol * np.linalg.norm(po[n]) + upd_tol * np.linalg.norm(po[n] - w_old)
            d = np.linalg.norm(pg[n].astype(np.float64) - po[n])
            assert d <= bound, (s, n, d, bound)


@pytest.mark.parametrize("seed0", [0, 42])
def test_config1_fp32_two_steps(seed0):
    init_o, init_g, res = _run(CONFIG1, 2, 64, 0, 0, seed0, steps=2)
    _check(init_o, init_g, res, TOL_FP32, GRAD_FP32, UPD_FP32)


def test_config1_bf16_two_steps():
    init_o, init_g, res = _run(CONFIG1, 2, 64, 1, 0, 0, steps=2)
    _check(init_o, init_g, res, TOL_BF16, TOL_BF16, UPD_BF16)


@pytest.mark.parametrize("precision", [0, 1])
def test_wide_model(precision):
    init_o, init_g, res = _run(WIDE, 2, 256, precision, 256, 3, steps=2)
    if precision == 0:
        _check(init_o, init_g, res, TOL_FP32, GRAD_FP32, UPD_FP32)
    else:
        _check(init_o, init_g, res, TOL_BF16, TOL_BF16, UPD_BF16)


def test_step_is_deterministic():
    """Two models from the same seed and batch give bit-identical losses,
    gradients and weights (no float atomics anywhere on the step)."""
    import gpu_util as gu
    from autoresearch_amd.model import GPT, GPTConfig
    outs = []
    for _ in range(2):
        gm = GPT(GPTConfig(**WIDE), 2, 256, precision=1, rope_period=256)
        gm.init_weights(5)
        x, y = _tokens(9, 2, 256, WIDE["vocab_size"])
        loss = gm.train_step(gu.dev(x), gu.dev(y), 0.0)
        outs.append((loss, gu.host(gm.params()).copy()))
        gm.close()
    assert outs[0][0] == outs[1][0]
    np.testing.assert_array_equal(outs[0][1], outs[1][1])


def test_training_reduces_loss():
    """test_training.mojo:148-158 behaviour: loss falls and stays finite over
    10 steps on a fixed batch (AdamW + Muon, bf16 compute)."""
    import gpu_util as gu
    from autoresearch_amd.model import GPT, GPTConfig
    gm = GPT(GPTConfig(**WIDE), 2, 256, precision=1, rope_period=256)
    gm.init_weights(42)
    x, y = _tokens(1, 2, 256, WIDE["vocab_size"])
    xd, yd = gu.dev(x), gu.dev(y)
    losses = [gm.train_step(xd, yd, 0.0) for _ in range(10)]
    gm.close()
    assert all(np.isfinite(losses))
    assert losses[0] < 3 * np.log(WIDE["vocab_size"])  # test_forward.mojo:114-120
    assert losses[-1] < losses[0]
