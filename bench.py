#!/usr/bin/env python3
"""Benchmark: training tokens/s of the full GPT training step on one MI355X.

Workload: depth 8, d_model 512, 4 heads x 128,
vocab 8192, T = 2048, B = 32, SSSL windows (1024 x3, 2048), ReLU^2 MLP,
value embeddings, softcap 15, Muon (5 Polar Express iterations) on every 2-D
matrix and AdamW on embeddings and scalars; bf16 matrix-core compute with
fp32 master weights.  Token ids are Zipf(1.1) over the vocabulary from seed 0
(synthetic; no dataset).  Weights follow the reference init (seed 42).
`--config 5` runs BASELINE config 5 instead (depth 12, d_model 768, 6 heads,
B = 64, same architecture), reported with the same fields.

A "step" = zero_grads -> forward -> backward -> AdamW + Muon update
(train.mojo:231-282), all on the GPU through the C ABI (--graph: replayed
from a HIP graph, ar_gpt_train_step_graph, bit-identical).  W untimed warm-up
steps, then exactly K steps between two device synchronisations.

Prints ONE JSON line.  `roofline` describes the dominant kernel class
(largest share of step time): HIP events bracket each GEMM / attention / Muon
launch on the model's stream during P further profiled steps, which run the
same kernels on the same stream right after the timed ones (events are kept
out of the timed steps, where they would add ~2 % of launch overhead);
`cpu_baseline` times the fp32 CPU oracle on this host on a bounded sample of
the same workload.  The default run (config 4, bf16) also reports, under
`extra_workloads`, short runs (2 warm-up + 5 timed + 2 profiled steps) of
config 4 at the reference's fp32 precision and of config 5 in bf16.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2516.6   # dense bf16 MFMA, MI355X
PEAK_FP32_TFLOPS = 157.3    # fp32 matrix, MI355X
METRIC = "training tokens/sec @ depth8 d512 T2048 (1 GPU) + MFMA util %"
CLASS_NAMES = ["linear_fwd", "linear_bwd_dx", "linear_bwd_dw", "flash_attn_fwd", "flash_attn_bwd_dq",
               "flash_attn_bwd_dkv", "muon_polar_express"]


def zipf_tokens(n: int, V: int, s: float, seed: int) -> np.ndarray:
    """Inverse-CDF Zipf: p_k ~ (k+1)^-s, k < V."""
    p = 1.0 / np.arange(1, V + 1, dtype=np.float64) ** s
    cdf = np.cumsum(p / p.sum())
    u = np.random.default_rng(seed).random(n)
    return np.minimum(np.searchsorted(cdf, u, side="right"), V - 1).astype(np.int64)


def step_flops(L, C, V, B, T, H, hd, windows, mats) -> float:
    """Algorithmic FLOPs of one training step (2 flop per multiply-add; backward = 2x forward):
    GEMMs 72*L*M*C^2 + 6*M*C*V, attention 14*B*H*hd*sum_layers sum_q keys(q),
    Muon 5*sum(4*l*s^2 + 2*s^3)."""
    M = B * T
    gemm = 72.0 * L * M * C * C + 6.0 * M * C * V
    attn = 0.0
    for ws in windows:
        keys = sum((q - max(0, q - ws) + 1) if ws > 0 else (q + 1) for q in range(T))
        attn += 14.0 * B * H * hd * keys
    muon = sum(5.0 * (4.0 * max(r, c) * min(r, c) ** 2 + 2.0 * min(r, c) ** 3) for r, c in mats)
    return gemm + attn + muon


def measured_traffic(cls: str, a, bf16: bool, depth: int, batch: int):
    """HBM bytes per launch of kernel class `cls` from the committed counter
    passes (rocprofv3 FETCH_SIZE / WRITE_SIZE, scaled by a 1 GiB copy; see
    profiles/counters_config4_bf16.md), for the workload those passes ran."""
    path = os.path.join(ROOT, "profiles", "traffic_config4_bf16.json")
    if not (bf16 and (depth, batch, a.seq, a.vocab) == (8, 32, 2048, 8192) and os.path.exists(path)):
        return None
    with open(path) as f:
        return json.load(f)["classes"].get(cls)


def cpu_model() -> str:
    """The host CPU's model name (what lscpu prints as "Model name")."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg, T, V, steps_tokens_B: int) -> dict:
    """fp32 CPU oracle on this host: one forward+backward at B=1 (2048 tokens)
    and one optimizer step, extrapolated to the B=32 step."""
    from oracle import oracle as orc
    om = orc.Model(cfg.as_dict(), 1, T, T)
    om.init_weights(42)
    toks = zipf_tokens(T + 1, V, 1.1, 1)
    x, y = np.ascontiguousarray(toks[:-1]), np.ascontiguousarray(toks[1:])
    t0 = time.perf_counter()
    om.zero_grads()
    om.forward(x, y)
    om.backward(x, y, 1.0)
    t1 = time.perf_counter()
    om.optimizer_step(0.0)
    t2 = time.perf_counter()
    fb, opt = t1 - t0, t2 - t1
    est = steps_tokens_B * fb + opt
    return {"value": round(steps_tokens_B * T / est, 2), "unit": "tokens/s",
            "cores": orc.lib().orc_num_threads(), "cpu_model": cpu_model(), "kind": "port",
            "sample": (f"fp32 oracle (OpenMP): 1 fwd+bwd at B=1,T={T} ({fb:.1f}s) + 1 AdamW/Muon update "
                       f"({opt:.1f}s), extrapolated to B={steps_tokens_B}: {steps_tokens_B}*fwdbwd + update")}


def vendor_comparator() -> list:
    """What the ROCm libraries reach on the step's shapes (config 4, bf16
    operands): hipBLASLt through torch.mm for each linear layer's forward
    (bf16 and fp32 output), dW and dX, a 8192^3 square, and torch's
    scaled_dot_product_attention at BASELINE config 2.  A comparator only:
    the library never calls them.  Mean of 20 calls after 3 warm-up calls."""
    import torch
    import torch.nn.functional as F

    def timed(f, n=20):
        for _ in range(3):
            f()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            f()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    torch.manual_seed(0)
    rows = []

    def row(name, ms, flops):
        rows.append({"product": name, "us": round(ms * 1e3, 1), "tflops": round(flops / ms / 1e9, 1)})
        print(f"[comparator] {name}: {ms * 1e3:.1f} us", file=sys.stderr, flush=True)

    M = 65536
    for lname, n, k in (("q|k|v", 1536, 512), ("c_proj", 512, 512), ("c_fc", 2048, 512), ("mlp_proj", 512, 2048),
                        ("lm_head", 8192, 512)):
        a = torch.randn(M, k, device="cuda", dtype=torch.bfloat16)
        w = torch.randn(n, k, device="cuda", dtype=torch.bfloat16) * 0.02
        dy = torch.randn(M, n, device="cuda", dtype=torch.bfloat16)
        out = torch.empty(M, n, device="cuda", dtype=torch.bfloat16)
        fl = 2.0 * M * n * k
        row(f"{lname} fwd {M}x{n}x{k} bf16 out", timed(lambda: torch.mm(a, w.t(), out=out)), fl)
        row(f"{lname} fwd {M}x{n}x{k} fp32 out", timed(lambda: torch.mm(a, w.t(), out_dtype=torch.float32)), fl)
        row(f"{lname} dW {n}x{k} (reduction {M})", timed(lambda: torch.mm(dy.t(), a)), fl)
        row(f"{lname} dX {M}x{k} (reduction {n})", timed(lambda: torch.mm(dy, w)), fl)
        del a, w, dy, out
    a = torch.randn(8192, 8192, device="cuda", dtype=torch.bfloat16)
    b = torch.randn(8192, 8192, device="cuda", dtype=torch.bfloat16)
    row("square 8192x8192x8192", timed(lambda: a @ b, 10), 2.0 * 8192 ** 3)
    del a, b
    q = torch.randn(16, 4, 2048, 128, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    k_ = torch.randn_like(q, requires_grad=True)
    v = torch.randn_like(q, requires_grad=True)
    fl = 4.0 * 16 * 4 * 128 * (2048 * 2049 / 2)
    row("sdpa causal fwd B16 H4 T2048 hd128", timed(lambda: F.scaled_dot_product_attention(q, k_, v, is_causal=True)),
        fl)
    g = torch.randn(16, 4, 2048, 128, device="cuda", dtype=torch.bfloat16)
    row("sdpa causal fwd+bwd B16 H4 T2048 hd128",
        timed(lambda: torch.autograd.grad(F.scaled_dot_product_attention(q, k_, v, is_causal=True), (q, k_, v), g)),
        3.5 * fl)
    return rows


def gemm_sweep() -> list:
    """The persistent GEMM (ar_gemm_mixed, bf16 operands) on the step's
    product shapes at several reduction lengths: time(K) = fixed + K-loop,
    so the intercept is the per-tile cost that does not scale with K (the
    epilogue, pipeline fill) and the slope the k-loop's rate.  Mean of 20
    calls after 3 warm-up calls, timed with torch events."""
    import ctypes as ct
    import torch
    from autoresearch_amd import _lib, ops

    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    ws = ops.Workspace(1 << 30).bind()

    def timed(f, n=20):
        for _ in range(3):
            f()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            f()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    rows = []
    M = 65536
    for layout, N, Ks, cb in ((0, 2048, (256, 512, 1024, 2048, 4096), 1), (0, 512, (512, 2048, 4096), 0),
                              (2, 2048, (16384, 32768, 65536, 131072), 0)):
        for K in Ks:
            if layout == 0:  # C[M, N] = X[M, K] W[N, K]^T
                X = torch.randn(M, K, device="cuda").to(torch.bfloat16)
                W = (torch.randn(N, K, device="cuda") * 0.02).to(torch.bfloat16)
                C = torch.empty(M, N, device="cuda", dtype=torch.bfloat16 if cb else torch.float32)
                m, n, k = M, N, K
            else:  # dW[N, 512] += dY[K, N]^T X[K, 512]: K is the reduction (tokens)
                X = torch.randn(K, N, device="cuda").to(torch.bfloat16)
                W = torch.randn(K, 512, device="cuda").to(torch.bfloat16)
                C = torch.zeros(N, 512, device="cuda")
                m, n, k = K, N, 512

            def f():
                r = lib.ar_gemm_mixed(ct.c_void_p(st), layout, ct.c_void_p(C.data_ptr()), cb, ct.c_void_p(X.data_ptr()),
                                      1, ct.c_void_p(W.data_ptr()), 1, m, n, k, 1 if layout == 2 else 0)
                if r != 0:
                    raise RuntimeError(lib.ar_last_error().decode())
            ms = timed(f)
            fl = 2.0 * M * N * K if layout == 0 else 2.0 * K * N * 512
            name = (f"NT {M}x{N}x{K} {'bf16' if cb else 'fp32'} out" if layout == 0
                    else f"TN dW {N}x512, reduction {K}")
            rows.append({"product": name, "us": round(ms * 1e3, 1), "tflops": round(fl / ms / 1e9, 1)})
            print(f"[gemm-sweep] {name}: {ms * 1e3:.1f} us", file=sys.stderr, flush=True)
            del X, W, C
    ws.close()
    return rows


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=11)
    ap.add_argument("--config", type=int, choices=[4, 5], default=4,
                    help="BASELINE workload: 4 = depth 8 d512 B32 (the metric), 5 = depth 12 d768 B64")
    ap.add_argument("--depth", type=int, default=None)
    ap.add_argument("--batch", type=int, default=None)
    ap.add_argument("--seq", type=int, default=2048)
    ap.add_argument("--vocab", type=int, default=8192)
    ap.add_argument("--precision", choices=["bf16", "fp32"], default="bf16")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra-legs", action="store_true",
                    help="skip the short fp32 config-4 and bf16 config-5 runs reported beside the headline")
    ap.add_argument("--graph", action="store_true", help="replay the step from a HIP graph")
    ap.add_argument("--prof-steps", type=int, default=5, help="profiled steps after the timed ones")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run one device copy of MIB MiB (calibrates rocprofv3 byte counters) and exit")
    ap.add_argument("--vendor-comparator", action="store_true",
                    help="only time hipBLASLt (torch.mm) and torch SDPA on the step's shapes and exit")
    ap.add_argument("--gemm-sweep", action="store_true",
                    help="only time the persistent GEMM over several reduction lengths and exit")
    a = ap.parse_args(argv)
    if a.depth is None:
        a.depth = 8 if a.config == 4 else 12
    if a.batch is None:
        a.batch = 32 if a.config == 4 else 64
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the training step is single-GPU in the reference; "
              "multi-GPU data parallelism is a design note, not built). Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    if a.vendor_comparator:
        print(json.dumps({"vendor_comparator": vendor_comparator()}), flush=True)
        return 0
    if a.gemm_sweep:
        print(json.dumps({"gemm_sweep": gemm_sweep()}), flush=True)
        return 0

    if a.copy_probe:
        n = a.copy_probe * (1 << 20) // 4
        src = torch.ones(n, device="cuda")
        dst = torch.empty(n, device="cuda")
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_read": 4 * n, "copy_probe_bytes_written": 4 * n}), flush=True)
        return 0

    torch.cuda.set_device(0)
    stream = torch.cuda.Stream()  # a stream of its own (graph capture cannot use the null stream)
    torch.cuda.set_stream(stream)
    head = run_workload(a, a.config, a.depth, a.batch, a.precision, a.steps, a.warmup, a.prof_steps, a.graph)
    cfg, B, T, V = head.pop("_cfg"), a.batch, a.seq, a.vocab

    # The other figures the driver should see beside the headline: config 4 at
    # the reference's own fp32 precision and config 5 in bf16 (short runs of
    # their own; the headline's timed region is unaffected).
    extra = {}
    if not a.no_extra_legs and (a.config, a.depth, a.batch, a.precision) == (4, 8, 32, "bf16"):
        for key, conf, depth, batch, prec in (("config4_fp32", 4, 8, 32, "fp32"), ("config5_bf16", 5, 12, 64, "bf16")):
            r = run_workload(a, conf, depth, batch, prec, 5, 2, 2, a.graph)
            r.pop("_cfg")
            extra[key] = {k: r[k] for k in ("workload", "dtype", "steps", "warmup", "ms_per_step", "value", "unit",
                                            "mfma_util", "roofline", "kernel_classes", "loss_after")}

    cpu = None
    if not a.no_cpu_baseline:
        print("[bench] cpu baseline (oracle) ...", file=sys.stderr, flush=True)
        cpu = cpu_baseline(cfg, T, V, B)

    out = {
        "metric": METRIC, "value": head["value"], "unit": "tokens/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": head["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": a.precision, "data": "synthetic Zipf(1.1) token ids, seed 0",
        "step_mode": "hip_graph" if a.graph else "eager",
        "config": {"workload": head["workload"], "global_batch": B, "seq_len": T, "parallelism": "single GPU"},
        "mfma_util": head["mfma_util"], "step_tflop": head["step_tflop"],
        "roofline": head["roofline"], "kernel_classes": head["kernel_classes"], "cpu_baseline": cpu,
        "loss_after": head["loss_after"],
    }
    if extra:
        out["extra_workloads"] = extra
    print(json.dumps(out), flush=True)
    return 0


def run_workload(a, config, depth, batch, precision, steps, warmup, prof_steps, graph) -> dict:
    """Build the model of one BASELINE workload, run W warm-up and K timed
    steps, then P event-profiled steps; return its figures."""
    import ctypes as ct
    import torch
    from autoresearch_amd._lib import check
    from autoresearch_amd.model import BF16, FP32, GPT, GPTConfig

    cfg = GPTConfig.default(a.vocab, depth)
    B, T, V = batch, a.seq, a.vocab
    prec = BF16 if precision == "bf16" else FP32
    toks = zipf_tokens(B * (T + 1), V, 1.1, 0).reshape(B, T + 1)
    x = torch.from_numpy(np.ascontiguousarray(toks[:, :-1]).ravel()).cuda()
    y = torch.from_numpy(np.ascontiguousarray(toks[:, 1:]).ravel()).cuda()
    m = GPT(cfg, B, T, precision=prec, rope_period=T)
    m.init_weights(42)
    torch.cuda.synchronize()
    print(f"[bench] model ready: L={cfg.n_layer} C={cfg.n_embd} H={cfg.n_head} V={V} B={B} T={T} "
          f"{precision} {'graph' if graph else 'eager'}", file=sys.stderr, flush=True)
    step = m.train_step_graph if graph else m.train_step

    for i in range(warmup):
        step(x, y, 0.0, sync_loss=False)
    torch.cuda.synchronize()
    print(f"[bench] warmup done ({warmup} steps)", file=sys.stderr, flush=True)

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(x, y, 0.0, sync_loss=False)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / steps

    # Per-class timing: HIP events around every GEMM / attention / Muon launch
    # of P eager steps on the same stream.
    check(m.lib.ar_gpt_profile(m.h, 1), "gpt_profile")
    for i in range(prof_steps):
        m.train_step(x, y, 0.0, sync_loss=False)
    cls_stats = []
    per = max(prof_steps, 1)
    for c in range(len(CLASS_NAMES)):
        t, n, f = ct.c_double(), ct.c_int64(), ct.c_double()
        check(m.lib.ar_gpt_profile_read(m.h, c, ct.byref(t), ct.byref(n), ct.byref(f)), "gpt_profile_read")
        cls_stats.append((CLASS_NAMES[c], t.value / per, n.value // per, f.value / per))
    check(m.lib.ar_gpt_profile(m.h, 0), "gpt_profile")
    torch.cuda.synchronize()
    loss = m.forward(x, y)
    print(f"[bench] timed {steps} steps: {ms:.2f} ms/step, loss after = {loss:.4f}", file=sys.stderr, flush=True)
    m.close()
    del x, y
    torch.cuda.empty_cache()

    value = B * T / (ms / 1e3)
    windows = [cfg.window_size(i) for i in range(cfg.n_layer)]
    mats = []
    F = 4 * cfg.n_embd
    for _ in range(cfg.n_layer):
        mats += [(cfg.n_embd, cfg.n_embd)] * 4 + [(F, cfg.n_embd), (cfg.n_embd, F)]
    flops = step_flops(cfg.n_layer, cfg.n_embd, V, B, T, cfg.n_head, cfg.head_dim, windows, mats)
    peak = PEAK_BF16_TFLOPS if prec == BF16 else PEAK_FP32_TFLOPS
    mfma_util = flops / (ms / 1e3) / (peak * 1e12)

    # per-step figures: (name, ms, launches, flops)
    dom = max(cls_stats, key=lambda s: s[1])
    name, t_ms, n, f = dom
    achieved = (f / (t_ms / 1e3)) / 1e12 if t_ms > 0 else 0.0
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                "frac": round(achieved / peak, 4),
                "traffic": measured_traffic(name, a, prec == BF16, depth, batch), "kernel": name,
                "launches_per_step": n, "avg_launch_ms": round(t_ms / max(n, 1), 4),
                "share_of_step": round(t_ms / ms, 4)}
    breakdown = {s[0]: {"ms_per_step": round(s[1], 3),
                        "tflops": round((s[3] / (s[1] / 1e3)) / 1e12, 1) if s[1] > 0 else 0.0}
                 for s in cls_stats}
    return {"_cfg": cfg, "workload": f"config {config}: full training step depth{cfg.n_layer} d{cfg.n_embd} "
                                     f"H{cfg.n_head}x{cfg.head_dim} V{V} T{T} B{B} SSSL, AdamW+Muon",
            "dtype": precision, "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 3),
            "value": round(value, 1), "unit": "tokens/s", "mfma_util": round(mfma_util, 4),
            "step_tflop": round(flops / 1e12, 3), "roofline": roofline, "kernel_classes": breakdown,
            "loss_after": round(loss, 4)}


if __name__ == "__main__":
    sys.exit(main())
