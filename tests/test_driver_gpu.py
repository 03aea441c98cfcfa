"""The ar_train driver (train.mojo:128-339) end to end on the GPU: a tiny
model on synthetic token shards, with --fake-dt fixing each step's time so the
schedule is deterministic.  Checks the log line and summary format, the time
budget / warm-up accounting, the LR schedule's closed form, that the first
logged loss is the library's forward loss on the first packed batch, and a
finite validation bits-per-byte."""
import math
import os
import re
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "autoresearch_amd", "ar_train")
STEP_RE = re.compile(r"^step (\d+)  \| (\d+) % \|  loss: (\S+)  \| lrm: (\S+)  \| dt: (\d+) ms  \| "
                     r"epoch: (\d+)  \| rem: (\d+) s$")
V, DEPTH, B, T, DT, BUDGET = 512, 2, 2, 64, 0.05, 1
_LOSSES = {}  # mode -> logged losses (graph replay must match the eager step exactly)


def _make_data(d):
    from autoresearch_amd import data
    rng = np.random.default_rng(11)

    def docs(n):
        out = []
        for _ in range(n):
            x = rng.integers(4, V, int(rng.integers(2, 200))).astype(np.int32)
            x[0] = 1
            out.append(x)
        return out
    data.write_shard(os.path.join(d, "shard_00000.tok"), docs(400), groups=[200, 200])
    data.write_shard(os.path.join(d, data.VAL_SHARD), docs(200))
    tb = rng.integers(1, 6, V).astype(np.int32)
    tb[:4] = 0  # special tokens carry no bytes
    data.write_token_bytes(os.path.join(d, "token_bytes.bin"), tb)


@pytest.mark.parametrize("graph", [False, True])
def test_driver_schedule_log_and_summary(tmp_path, graph):
    assert os.path.exists(DRIVER), "build the driver first (python -m autoresearch_amd.build)"
    d = str(tmp_path)
    _make_data(d)
    env = dict(os.environ, TRAIN_TIME_BUDGET=str(BUDGET))
    cmd = [DRIVER, "--data", d, "--tokenizer", d, "--vocab", str(V), "--depth", str(DEPTH), "--batch", str(B),
           "--seq", str(T), "--fake-dt", str(DT)] + (["--graph"] if graph else [])
    print("running", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=180)
    print(r.stdout[-3000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0
    lines = r.stdout.splitlines()
    assert f"Model: L= {DEPTH}  H= 1  C= 128  V= {V}" in lines
    assert f"Batch: B= {B}  T= {T}  tokens/step= {B * T}" in lines
    assert f"Time budget: {BUDGET} s" in lines
    steps = [STEP_RE.match(l) for l in lines if l.startswith("step ")]
    assert steps and all(steps)
    # expected step count: steps 0..10 are not timed, then DT per step until the budget
    tt, n = 0.0, 0
    while True:
        if n > 10:
            tt += DT
        n += 1
        if n > 10 and tt >= BUDGET:
            break
    assert len(steps) == n
    tt = 0.0
    losses = []
    for s, m in enumerate(steps):
        step, pct, loss, lrm, dt_ms, epoch, rem = m.groups()
        assert int(step) == s and int(dt_ms) == int(DT * 1000) and int(epoch) >= 1
        progress = min(1.0, tt / BUDGET)
        assert int(pct) == int(100 * progress)
        # warmdown schedule (config.mojo:81-83): 1 until progress 0.5, then 2 (1 - progress)
        want = 1.0 if progress < 0.5 else 2.0 * (1.0 - progress)
        assert abs(float(lrm) - want) <= 1e-12
        if s > 10:
            tt += DT
        assert int(rem) == int(max(0.0, BUDGET - tt))
        losses.append(float(loss))
    assert all(math.isfinite(x) for x in losses)
    assert losses[-1] < losses[0]  # the debiased smoothed loss falls
    _LOSSES[graph] = losses
    if len(_LOSSES) == 2:
        assert _LOSSES[True] == _LOSSES[False]
    # summary block (train.mojo:331-339)
    summ = dict(l.split(":", 1) for l in lines[lines.index("---") + 1:])
    assert [k for k in summ] == ["val_bpb", "training_seconds", "total_seconds", "startup_seconds",
                                 "total_tokens_M", "num_steps", "depth"]
    assert int(summ["num_steps"]) == n and int(summ["depth"]) == DEPTH
    assert abs(float(summ["training_seconds"]) - tt) < 1e-12
    assert abs(float(summ["total_tokens_M"]) - n * B * T / 1e6) < 1e-12
    bpb = float(summ["val_bpb"])
    assert math.isfinite(bpb) and 0.0 < bpb < 10.0

    # the first logged loss is the model's forward loss on the first packed batch
    import gpu_util as gu
    from autoresearch_amd import data
    from autoresearch_amd.model import GPT, GPTConfig
    x, y, _ = data.Loader(d, "train", B, T).next()
    gm = GPT(GPTConfig.default(V, DEPTH), B, T, precision=1, rope_period=0)
    gm.init_weights(42)
    l0 = gm.forward(gu.dev(x.ravel()), gu.dev(y.ravel()))
    gm.close()
    assert abs(losses[0] - l0) <= 1e-6 * abs(l0), (losses[0], l0)


@pytest.mark.parametrize("graph", [False, True])
def test_driver_nan_fast_fail(tmp_path, graph):
    """train.mojo:284-287: a NaN loss ends training with "FAIL: loss = nan"
    right after the step that produced it, before its log line, and no
    evaluation or summary follows.  The NaN is forced from the host
    (--nan-at writes one into lm_head before step 3); every kernel runs
    normally on the NaN data."""
    d = str(tmp_path)
    _make_data(d)
    env = dict(os.environ, TRAIN_TIME_BUDGET=str(BUDGET))
    cmd = [DRIVER, "--data", d, "--tokenizer", d, "--vocab", str(V), "--depth", str(DEPTH), "--batch", str(B),
           "--seq", str(T), "--fake-dt", str(DT), "--nan-at", "3"] + (["--graph"] if graph else [])
    print("running", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=180)
    print(r.stdout[-3000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0  # the reference returns from main
    lines = r.stdout.splitlines()
    steps = [STEP_RE.match(l) for l in lines if l.startswith("step ")]
    assert [int(m.group(1)) for m in steps] == [0, 1, 2]
    assert all(math.isfinite(float(m.group(3))) for m in steps)
    assert lines[-1] == "FAIL: loss = nan"
    assert "---" not in lines and not any(l.startswith("val_bpb") for l in lines)
