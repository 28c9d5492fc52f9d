"""kurumi_hip benchmark: the five headline configs on one MI355X, plus the CPU baseline.

The headline line (metric/value) is config 2 — row softmax over [8192, 32000] f32 built from
primitives (reduce_max, sub, exp, sum, div) followed by argmax -> int32 — as HBM GB/s of the
single fused kernel's algorithmic traffic. Every config runs as a device-resident plan
(inputs uploaded once, threefry-seeded synthetic data generated on the device), W untimed
launches, then K timed launches bracketed by hipEvents on the plan's own stream. The other
configs are reported under "configs" with their own roofline fractions and CPU baselines;
config "6" is the nn primitives around them (rope, the SwiGLU gate, rmsnorm, the int4
QuantMatmul). The `make_*` functions build exactly the plans that are timed; the full-size GPU
tests (tests/test_gpu_bench_configs.py) run those same plans and check their outputs.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs 1,2,3,4,5,6] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path
from types import SimpleNamespace

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2516.6
FP8_PEAK_TFLOPS = 5033.2


def _ku():
    import kurumi_amd as K

    return K


def device_values(hip, build, shape, seed, dtype):
    """Generate kurumi's seeded random tensor on the device (threefry2x32 inside the graph)."""
    K = _ku()
    g = K.Graph()
    x = build(g, list(shape), seed)
    if dtype != K.DType.F32:
        x = g.cast(x, dtype)
    return hip.eval(g, x)


def scaled_randn(std):
    return lambda g, s, sd: g.mul(g.randn(s, sd), g.expand(g.constant(np.array([std], np.float32).reshape(
        [1] * len(s))), s))


def uniform_pm1(g, s, sd):
    return g.rand_range(s, sd, -1.0, 1.0)


# ---------------- the graphs and plans that are timed ----------------

def softmax_graph(K, rows, cols, dt):
    """cfg 2: softmax from primitives (reduce_max, sub, exp, sum, div), then argmax -> i32."""
    g = K.Graph()
    x = g.input([rows, cols], dt)
    m = g.reduce_max(x, 1)
    e = g.exp(g.sub(x, g.expand(g.reshape(m, [rows, 1]), [rows, cols])))
    s = g.sum(e, 1)
    y = g.div(e, g.expand(g.reshape(s, [rows, 1]), [rows, cols]))
    a = g.cast(g.argmax(y, 1), K.DType.I32)
    return g, x, y, a


def cfg1_graph(K, n):
    """cfg 1: sum over the last axis of relu(x*x + b) * 0.5."""
    g = K.Graph()
    x = g.input([n, n], K.DType.F32)
    b = g.input([n], K.DType.F32)
    h = g.mul(g.relu(g.add(g.mul(x, x), g.broadcast_to(b, [n, n]))), g.scalar(x, 0.5))
    return g, x, b, g.sum(h, 1)


def make_cfg1(hip, rep=0):
    K = _ku()
    n = 4096
    g, x, b, y = cfg1_graph(K, n)
    xt = device_values(hip, uniform_pm1, [n, n], 100 + rep, K.DType.F32)
    bt = device_values(hip, uniform_pm1, [n], 200 + rep, K.DType.F32)
    feeds = {x: xt, b: bt}
    return SimpleNamespace(plan=hip.plan(g, [y], feeds), g=g, x=x, b=b, roots=[y], feeds=feeds,
                           algo_bytes=4 * n * n + 4 * n + 4 * n)


def make_cfg2(hip, dt_name="f32"):
    K = _ku()
    rows, cols = 8192, 32000
    dt = K.DType.F32 if dt_name == "f32" else K.DType.BF16
    xt = device_values(hip, scaled_randn(3.0), [rows, cols], 2024, dt)
    g, x, y, a = softmax_graph(K, rows, cols, dt)
    feeds = {x: xt}
    w = 4 if dt == K.DType.F32 else 2
    return SimpleNamespace(plan=hip.plan(g, [y, a], feeds), g=g, x=x, y=y, a=a, roots=[y, a], feeds=feeds,
                           rows=rows, cols=cols, dt=dt,
                           algo_bytes=rows * cols * w * 2 + rows * 4)  # read x, write y, write i32 argmax


def gemm_graph(K, batched):
    g = K.Graph()
    if batched:
        sa, sb, std = [8, 2048, 128], [8, 128, 2048], 1.0 / np.sqrt(128)
        a = g.input(sa, K.DType.BF16)
        b = g.input(sb, K.DType.BF16)
        c = g.dot_general(a, b, [2], [1], [0], [0])
        flops = 2 * 8 * 2048 * 2048 * 128
    else:
        sa, sb, std = [4096, 4096], [4096, 11008], 1.0 / 64
        a = g.input(sa, K.DType.BF16)
        b = g.input(sb, K.DType.BF16)
        c = g.matmul(a, b)
        flops = 2 * 4096 * 4096 * 11008
    return g, a, b, c, sa, sb, std, flops


def make_gemm(hip, batched=False, rep=0):
    K = _ku()
    g, a, b, c, sa, sb, std, flops = gemm_graph(K, batched)
    at = device_values(hip, scaled_randn(std), sa, 301 + 10 * rep, K.DType.BF16)
    bt = device_values(hip, scaled_randn(std), sb, 302 + 10 * rep, K.DType.BF16)
    feeds = {a: at, b: bt}
    byts = 2 * (int(np.prod(sa)) + int(np.prod(sb))) + 2 * (int(np.prod(sa[:-1])) * sb[-1])
    return SimpleNamespace(plan=hip.plan(g, [c], feeds), g=g, a=a, b=b, c=c, roots=[c], feeds=feeds,
                           flops=flops, algo_bytes=byts)


def make_attention(hip):
    K = _ku()
    B, H, S, D = 4, 32, 2048, 128
    g = K.Graph()
    q = g.input([B, H, S, D], K.DType.BF16)
    k = g.input([B, H, S, D], K.DType.BF16)
    v = g.input([B, H, S, D], K.DType.BF16)
    o = g.sdpa(q, k, v, True)
    feeds = {n: device_values(hip, lambda gg, s, sd: gg.randn(s, sd), [B, H, S, D], 400 + i, K.DType.BF16)
             for i, n in enumerate([q, k, v])}
    return SimpleNamespace(plan=hip.plan(g, [o], feeds), g=g, q=q, k=k, v=v, o=o, roots=[o], feeds=feeds,
                           flops=4 * B * H * S * S * D // 2, algo_bytes=4 * B * H * S * D * 2)


def fp8_graph(K, x_shape, w_f32: bytes, w_shape):
    """cfg 5: a bf16 linear x @ W^T with an f32 weight constant, through the e4m3 pass (which
    quantizes W per row from its stored f32 values and x per tensor in the graph)."""
    g = K.Graph()
    x = g.input(list(x_shape), K.DType.BF16)
    w = g.constant_bytes(K.DType.F32, w_f32, list(w_shape))
    y0 = g.dot_general(x, g.cast(w, K.DType.BF16), [1], [1])
    return g, x, K.amp_fp8(g, y0)


def make_fp8(hip):
    K = _ku()
    M, Kd, N = 2048, 4096, 11008
    wt = device_values(hip, scaled_randn(0.02), [N, Kd], 501, K.DType.F32)
    g, x, y = fp8_graph(K, [M, Kd], wt.data, [N, Kd])
    xt = device_values(hip, lambda gg, s, sd: gg.randn(s, sd), [M, Kd], 502, K.DType.BF16)
    feeds = {x: xt}
    # Xq + Wq + sw + Y (bf16): the GEMM's algorithmic bytes
    return SimpleNamespace(plan=hip.plan(g, [y], feeds), g=g, x=x, y=y, roots=[y], feeds=feeds, w=wt,
                           M=M, K=Kd, N=N, flops=2 * M * N * Kd, algo_bytes=M * Kd + N * Kd + 4 * N + 2 * M * N)


# ---------------- timing ----------------

# The extra configs run after host-side set-up (input generation, planning, uploads) during
# which the GPU idles and its clocks drop; they take at least this much warm-up work (besides
# --warmup launches) so each is timed at the clocks it holds under load. The headline takes
# exactly --warmup launches.
EXTRA_WARM_MS = 100.0


def time_plans(plans, steps: int, warmup: int, use_graph: bool = False, warm_ms: float = EXTRA_WARM_MS):
    """Warm up, then the timed region: `steps` rounds, each launching every plan once (rotating
    independent input sets), bracketed by hipEvents on the plans' stream and by a host clock
    around the call, which ends with the stream drained. Returns (wall ms per launch, GPU ms of
    each step of a launch, step labels): the GPU time per launch comes from the timed region's
    events; for a multi-kernel plan a following run with events between the steps splits it.
    Warm-up: `warmup` rounds, then more rounds until `warm_ms` of wall time has passed."""
    K = _ku()
    for _ in range(warmup):
        for p in plans:
            p.launch(use_graph)
    plans[0].sync()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < warm_ms:
        for _ in range(10):
            for p in plans:
                p.launch(use_graph)
        plans[0].sync()
    t0 = time.perf_counter()
    gpu_ms = K.time_plans(plans, steps, use_graph) / len(plans)
    wall_ms = (time.perf_counter() - t0) * 1e3 / (steps * len(plans))
    labels = plans[0].steps()
    if len(labels) == 1:
        return wall_ms, [gpu_ms], labels
    shares = plans[0].time_steps(max(steps, 5))
    tot = sum(shares)
    per_step = [s / tot * gpu_ms for s in shares] if tot > 0 else shares
    return wall_ms, per_step, labels


def measured_traffic(kernel: str):
    """HBM bytes per launch of a kernel, from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    passes (profiles/hbm_traffic.json, scaled by the copy-kernel calibration). Keyed by the
    kernel's plan label (generated kernels hash their source into it): a changed kernel reads
    as null."""
    path = ROOT / "profiles" / "hbm_traffic.json"
    if not path.exists() or not kernel:
        return None
    rec = json.loads(path.read_text()).get("kernels", {}).get(kernel)
    return rec["traffic_bytes"] if rec else None


def roofline_hbm(bytes_per_launch: float, kernel_ms: float, kernel: str | None = None):
    gbs = bytes_per_launch / (kernel_ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(kernel)}


def roofline_mfma(flops: float, kernel_ms: float, peak_tflops: float, kernel: str | None = None):
    tf = flops / (kernel_ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": round(tf, 1), "peak": peak_tflops, "unit": "TFLOP/s",
            "frac": round(tf / peak_tflops, 4), "traffic": measured_traffic(kernel)}


def main_kernel(per_step, labels, prefix):
    i = next(i for i, l in enumerate(labels) if l.startswith(prefix))
    return per_step[i], labels[i]


# ---------------- configs ----------------

def bench_cfg2(hip, steps, warmup, dt_name="f32"):
    c = make_cfg2(hip, dt_name)
    # the headline (f32) takes exactly --warmup launches
    wall_ms, per_step, labels = time_plans([c.plan], steps, warmup, warm_ms=0.0 if dt_name == "f32" else EXTRA_WARM_MS)
    kms = max(per_step)
    k = per_step.index(kms)
    out = {
        "workload": f"softmax+argmax [{c.rows},{c.cols}] {dt_name} (decomposed primitives)",
        "ms_per_step": wall_ms, "kernels": labels, "kernel_ms": per_step, "dominant": labels[k],
        "algo_bytes": c.algo_bytes, "value_gbs": c.algo_bytes / (wall_ms * 1e-3) / 1e9,
        "roofline": roofline_hbm(c.algo_bytes, kms, labels[k]),
    }
    if dt_name == "f32":
        # the same plan replayed as one hipGraph per launch (the ku_plan_run path)
        gw, gper, _ = time_plans([c.plan], steps, warmup, use_graph=True, warm_ms=0.0)
        out["graph_replay"] = {"ms_per_step": gw, "kernel_ms": gper[0],
                               "gbs": c.algo_bytes / (gper[0] * 1e-3) / 1e9}
    out["_cfg"] = c
    return out


def bench_cfg1(hip, steps, warmup):
    # 5 rotating input sets (5 x 64 MiB > the 256 MiB last-level cache): the kernel streams from HBM
    cs = [make_cfg1(hip, r) for r in range(5)]
    wall_ms, per_step, labels = time_plans([c.plan for c in cs], steps, warmup)
    return {"workload": "sum_lastaxis(relu(x*x+b)*0.5) [4096,4096] f32, 5 rotating input sets",
            "ms_per_step": wall_ms, "kernels": labels, "kernel_ms": per_step, "algo_bytes": cs[0].algo_bytes,
            "roofline": roofline_hbm(cs[0].algo_bytes, per_step[0], labels[0]), "_cfg": cs[0]}


def bench_gemm(hip, steps, warmup, batched=False):
    # the batched case (75 MB per set) rotates 4 input sets past the 256 MB last-level cache
    cs = [make_gemm(hip, batched, r) for r in range(4 if batched else 1)]
    wall_ms, per_step, labels = time_plans([c.plan for c in cs], steps, warmup)
    kms, kl = main_kernel(per_step, labels, "gemm")
    c = cs[0]
    out = {"workload": ("batched [8,2048,128]@[8,128,2048]" if batched else "[4096,4096]@[4096,11008]") + " bf16"
                       + (", 4 rotating input sets" if batched else ""),
           "ms_per_step": wall_ms, "kernels": labels, "kernel_ms": per_step, "flops": c.flops,
           "algo_bytes": c.algo_bytes, "roofline": roofline_mfma(c.flops, kms, BF16_PEAK_TFLOPS, kl), "_cfg": c}
    if batched:
        out["roofline_hbm"] = roofline_hbm(c.algo_bytes, kms, kl)
    return out


def bench_attention(hip, steps, warmup):
    c = make_attention(hip)
    wall_ms, per_step, labels = time_plans([c.plan], steps, warmup)
    return {"workload": "causal sdpa B4 H32 S2048 D128 bf16 (Op::Sdpa via g.sdpa)", "ms_per_step": wall_ms,
            "kernels": labels, "kernel_ms": per_step, "flops": c.flops,
            "roofline": roofline_mfma(c.flops, max(per_step), BF16_PEAK_TFLOPS, labels[0]), "_cfg": c}


def bench_fp8(hip, steps, warmup):
    c = make_fp8(hip)
    wall_ms, per_step, labels = time_plans([c.plan], steps, warmup)
    gemm_ms, gl = main_kernel(per_step, labels, "gemm")
    step_ms = sum(per_step)
    return {"workload": "e4m3 linear X[2048,4096] W[11008,4096]^T per-row/per-tensor scales, bf16 out",
            "ms_per_step": wall_ms, "kernels": labels, "kernel_ms": per_step, "flops": c.flops,
            "roofline": roofline_mfma(c.flops, gemm_ms, FP8_PEAK_TFLOPS, gl),
            "end_to_end": {"kernel_ms": step_ms, "tflops": round(c.flops / (step_ms * 1e-3) / 1e12, 1),
                           "frac": round(c.flops / (step_ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4)},
            "_cfg": c}


def bench_nn(hip, steps, warmup):
    """The nn primitives around the configs: rope (f32, the cfg 4 q shape), the SwiGLU gate
    silu(a) * b (bf16, the cfg 3 MLP shape) and rmsnorm (bf16, the cfg 2 row count). Each is
    HBM-bound; the gate and rmsnorm run three independent replicas per plan so the working set
    (3 x 135 MB) exceeds the 256 MB last-level cache, and their time per launch is the plan's
    GPU time over the replicas."""
    K = _ku()
    out = {}
    shp = [4, 32, 2048, 128]
    g = K.Graph()
    feeds, roots = {}, []
    for r in range(2):  # two replicas: 2 x (134 MB in + 134 MB out) > the last-level cache
        x = g.input(shp, K.DType.F32)
        feeds[x] = device_values(hip, scaled_randn(1.0), shp, 401 + r, K.DType.F32)
        roots.append(g.rope(x))
    plan = hip.plan(g, roots, feeds)
    wall_ms, per_step, labels = time_plans([plan], steps, warmup)
    main = [i for i, l in enumerate(labels) if l.startswith("ku_ew_4x32x2048x128")]
    kms = sum(per_step[i] for i in main) / len(main)
    n = int(np.prod(shp))
    algo = 8 * n + 2 * 2048 * 64 * 4  # read x, write y, read the two [S, D/2] tables
    out["nn_rope"] = {"workload": "rope [4,32,2048,128] f32 (table kernel + one fused kernel), 2 replicas per plan",
                      "ms_per_step": wall_ms / 2, "kernels": labels, "kernel_ms": per_step, "algo_bytes": algo,
                      "roofline": roofline_hbm(algo, kms, labels[main[0]])}
    reps = 3
    for name, shape, build, bytes_per in (
            ("nn_swiglu", [2048, 11008], lambda gg, ins: gg.mul(gg.silu(ins[0]), ins[1]), 3 * 2),
            ("nn_rmsnorm", [8192, 4096], lambda gg, ins: gg.rmsnorm(ins[0], 1, 1e-6), 2 * 2)):
        g = K.Graph()
        feeds, roots = {}, []
        for r in range(reps):
            ins = [g.input(shape, K.DType.BF16) for _ in range(2 if name == "nn_swiglu" else 1)]
            for i, t in enumerate(ins):
                feeds[t] = device_values(hip, scaled_randn(2.0), shape, 500 + 10 * r + i, K.DType.BF16)
            roots.append(build(g, ins))
        plan = hip.plan(g, roots, feeds)
        wall_ms, per_step, labels = time_plans([plan], steps, warmup)
        kms = sum(per_step) / reps
        algo = bytes_per * int(np.prod(shape))
        out[name] = {"workload": ("silu(a) * b" if name == "nn_swiglu" else "rmsnorm(x, axis 1, 1e-6)") +
                     f" {shape} bf16, {reps} independent replicas per plan",
                     "ms_per_step": wall_ms / reps, "kernels": labels, "kernel_ms": per_step, "algo_bytes": algo,
                     "roofline": roofline_hbm(algo, kms, labels[0])}
    return out


def bench_quant(hip, steps, warmup):
    """Weight-only int4 QuantMatmul through a [11008, 4096] int4 projection (symmetric, group 128,
    bf16 activations) per layer, 12 layers' weights per plan (12 x 23 MB exceeds the 256 MB
    last-level cache): one token (M = 1, the fused dequant GEMV) and a batch of 32 tokens (the
    fused dequant MFMA kernel). Both HBM-bound on the packed weights + scales."""
    K = _ku()
    n, k, grp, layers = 11008, 4096, 128, 12
    rng = np.random.default_rng(0)
    weights = []
    for _ in range(layers):
        w = rng.standard_normal((n, k), dtype=np.float32)
        packed, scales, _ = K.quantize(w, 4, grp, True)
        weights.append((packed, scales))
    out = {}
    for m, key, what in ((1, "nn_quant_gemv", "decode GEMV"), (32, "nn_quant_mfma", "batched decode (fused MFMA)")):
        g = K.Graph()
        x = g.input([m, k], K.DType.BF16)
        roots = []
        for packed, scales in weights:
            qw = g.constant_bytes(K.DType.U8, packed.tobytes(), packed.shape)
            sc = g.constant_bytes(K.DType.F16, scales.tobytes(), scales.shape)
            roots.append(g.quant_matmul(x, qw, sc, None, 4, grp))
        xt = device_values(hip, scaled_randn(1.0), [m, k], 601, K.DType.BF16)
        plan = hip.plan(g, roots, {x: xt})
        wall_ms, per_step, labels = time_plans([plan], steps, warmup)
        kms = sum(per_step) / layers
        algo = n * k // 2 + n * (k // grp) * 2 + m * k * 2 + m * n * 2  # packed weight, scales, act, out
        out[key] = {"workload": f"int4 (sym, group {grp}) {what} [{m},{k}] x [{n},{k}]^T bf16, "
                               f"{layers} layers' weights per plan", "ms_per_step": wall_ms / layers,
                    "kernels": labels[:1], "kernel_ms": per_step[:1], "algo_bytes": algo,
                    "roofline": roofline_hbm(algo, kms, labels[0])}
    return out


def bench_copy(hip, steps, warmup):
    """A plain streaming copy of 2^28 f32 (1 GiB read + 1 GiB write) through a one-leaf region."""
    K = _ku()
    n = 1 << 28
    g = K.Graph()
    x = g.input([n // 4096, 4096], K.DType.F32)
    y = g.neg(g.neg(x))
    xt = device_values(hip, lambda gg, s, sd: gg.rand_uniform(s, sd), [n // 4096, 4096], 7, K.DType.F32)
    plan = hip.plan(g, [y], {x: xt})
    wall_ms, per_step, labels = time_plans([plan], steps, warmup)
    return {"workload": "copy 1 GiB f32 (y = -(-x))", "kernels": labels, "kernel_ms": per_step,
            "algo_bytes": 2 * 4 * n, "roofline": roofline_hbm(2 * 4 * n, max(per_step), labels[0])}


# ---------------- CPU baselines (the oracle: single-threaded C++ restatement of kurumi's CPU paths) ----------------

def _oracle():
    sys.path.insert(0, str(ROOT / "tests"))
    import kutest

    return kutest


def _time_cpu(run, budget_s, max_reps=20):
    """Average seconds of `run()` (the oracle call alone: it returns raw output handles, released
    outside the timed span) with this thread pinned to one core, so the figure is single-core
    whatever threads the call starts (they inherit the affinity). The affinity is restored after."""
    kt = _oracle()
    saved = os.sched_getaffinity(0)
    os.sched_setaffinity(0, {min(saved)})
    try:
        kt.free_raw(run())  # warm-up
        reps, total = 0, 0.0
        while True:
            t0 = time.perf_counter()
            out = run()
            total += time.perf_counter() - t0
            kt.free_raw(out)
            reps += 1
            if total > budget_s or reps >= max_reps:
                return total / reps, reps
    finally:
        os.sched_setaffinity(0, saved)


def _cpu_line(value, unit, sample, reps, sec):
    return {"value": value, "unit": unit, "cores": 1, "kind": "port",
            "sample": f"{sample}; {reps} reps, {sec * 1e3:.1f} ms/rep; pinned to one core of host "
                      f"nproc={os.cpu_count()}; inputs bound and outputs released outside the timed call"}


def cpu_baseline_cfg2(xt_full, dt_name="f32", rows_sample=None, cols=32000):
    """The oracle interpreter on a row sample of the same logits (rows are independent), about
    10 s of single-core work: f32 through the decomposed primitives, bf16 through the same chain
    with the interpreter's per-primitive bf16 rounding (interp/elementwise.rs, interp/nn.rs:18-33)."""
    kt, K = _oracle(), _ku()
    bf16 = dt_name == "bf16"
    rows_sample = rows_sample or (256 if bf16 else 1024)
    dt = K.DType.BF16 if bf16 else K.DType.F32
    xs = np.ascontiguousarray(xt_full.numpy()[:rows_sample])
    g, x, y, a = softmax_graph(K, rows_sample, cols, dt)
    f = K.Feeds({x: K.Tensor(dt, [rows_sample, cols], xs.tobytes())})
    sec, reps = _time_cpu(lambda: kt.interpret_raw(g, [y, a], f), 10.0)
    w = 2 if bf16 else 4
    algo_bytes = rows_sample * cols * 2 * w + rows_sample * 4
    return _cpu_line(round(algo_bytes / sec / 1e9, 4), "GB/s",
                     f"{rows_sample} of 8192 rows x 32000 {dt_name}, decomposed softmax + argmax via the oracle "
                     f"interpreter", reps, sec)


def cpu_baseline_cfg1(c):
    """The view-fused CPU path (restated realize::force) on the full cfg 1 input."""
    kt, K = _oracle(), _ku()
    f = K.Feeds(c.feeds)
    sec, reps = _time_cpu(lambda: kt.realize_raw(c.g, c.roots[0], f), 4.0)
    return _cpu_line(round(c.algo_bytes / sec / 1e9, 4), "GB/s",
                     "full [4096,4096] f32 through the view-fused realize path", reps, sec)


def cpu_baseline_gemm(c, batched):
    """The oracle interpreter's contraction on a stated sub-shape (f32 accumulate, bf16 out),
    reported as GFLOP/s of that sub-shape (the work is linear in the rows)."""
    kt, K = _oracle(), _ku()
    g = K.Graph()
    if batched:
        sa, sb = [1, 256, 128], [1, 128, 2048]
        a, b = g.input(sa, K.DType.BF16), g.input(sb, K.DType.BF16)
        y = g.dot_general(a, b, [2], [1], [0], [0])
        src_a = c.feeds[c.a].numpy()[:1, :256]
        src_b = c.feeds[c.b].numpy()[:1]
    else:
        sa, sb = [8, 4096], [4096, 11008]
        a, b = g.input(sa, K.DType.BF16), g.input(sb, K.DType.BF16)
        y = g.matmul(a, b)
        src_a = c.feeds[c.a].numpy()[:8]
        src_b = c.feeds[c.b].numpy()
    feeds = {a: K.Tensor(K.DType.BF16, sa, np.ascontiguousarray(src_a).tobytes()),
             b: K.Tensor(K.DType.BF16, sb, np.ascontiguousarray(src_b).tobytes())}
    f = K.Feeds(feeds)
    sec, reps = _time_cpu(lambda: kt.interpret_raw(g, [y], f), 4.0, 5)
    flops = 2 * int(np.prod(sa)) * sb[-1]
    return _cpu_line(round(flops / sec / 1e9, 4), "GFLOP/s",
                     f"{sa}@{sb} bf16 (sub-shape of the config) via the oracle interpreter", reps, sec)


def cpu_baseline_attention(c):
    """The oracle's sdpa on one of the 128 (batch, head) slices, causal."""
    kt, K = _oracle(), _ku()
    S, D = 2048, 128
    g = K.Graph()
    q, k, v = (g.input([1, 1, S, D], K.DType.BF16) for _ in range(3))
    o = g.sdpa_fused(q, k, v, True)
    feeds = {n: K.Tensor(K.DType.BF16, [1, 1, S, D], np.ascontiguousarray(c.feeds[src].numpy()[:1, :1]).tobytes())
             for n, src in ((q, c.q), (k, c.k), (v, c.v))}
    f = K.Feeds(feeds)
    sec, reps = _time_cpu(lambda: kt.interpret_raw(g, [o], f), 4.0, 3)
    flops = 4 * S * S * D // 2
    return _cpu_line(round(flops / sec / 1e9, 4), "GFLOP/s",
                     "one (batch, head) slice [1,1,2048,128] bf16 causal via the oracle interpreter", reps, sec)


def cpu_baseline_fp8(c, rows=8):
    """The oracle interpreter on the e4m3 graph with `rows` activation rows."""
    kt, K = _oracle(), _ku()
    g, x, y = fp8_graph(K, [rows, c.K], c.w.data, [c.N, c.K])
    feeds = {x: K.Tensor(K.DType.BF16, [rows, c.K], np.ascontiguousarray(c.feeds[c.x].numpy()[:rows]).tobytes())}
    f = K.Feeds(feeds)
    sec, reps = _time_cpu(lambda: kt.interpret_raw(g, [y], f), 4.0, 5)
    flops = 2 * rows * c.N * c.K
    return _cpu_line(round(flops / sec / 1e9, 4), "GFLOP/s",
                     f"[{rows},{c.K}] x [{c.N},{c.K}]^T e4m3 linear (sub-shape) via the oracle interpreter", reps, sec)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 20 warm-up launches bring the clocks up (3 left the bf16 softmax 5-15 % slow on some runs)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--configs", default="1,2,3,4,5,6")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--probe-copy", action="store_true",
                    help="also run a plain 1 GiB f32 copy kernel (counter calibration / copy ceiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"kurumi_hip bench: this run measures one GPU only; --gpus {args.gpus} is not supported "
              "(every config shards with no exchange step)", file=sys.stderr)
        return 2
    K = _ku()
    hip = K.HipBackend()
    cfgs = {c.strip() for c in args.configs.split(",") if c.strip()}
    head = bench_cfg2(hip, args.steps, args.warmup, "f32")
    hc = head.pop("_cfg")
    extra = {}
    if "2" in cfgs:
        extra["cfg2_bf16"] = bench_cfg2(hip, args.steps, args.warmup, "bf16")
    if "1" in cfgs:
        extra["cfg1"] = bench_cfg1(hip, args.steps, args.warmup)
    if "3" in cfgs:
        extra["cfg3"] = bench_gemm(hip, args.steps, args.warmup)
        extra["cfg3b"] = bench_gemm(hip, args.steps, args.warmup, batched=True)
    if "4" in cfgs:
        extra["cfg4"] = bench_attention(hip, args.steps, args.warmup)
    if "5" in cfgs:
        extra["cfg5"] = bench_fp8(hip, args.steps, args.warmup)
    if "6" in cfgs:
        extra.update(bench_nn(hip, args.steps, args.warmup))
        extra.update(bench_quant(hip, args.steps, args.warmup))
    if args.probe_copy:
        extra["copy_probe"] = bench_copy(hip, args.steps, args.warmup)
    # the same step through the host boundary (ku_eval_many with host feeds -> host results):
    # PCIe-inclusive rate, reported beside the device-resident value (last: the GPU idles while
    # the host copies, which would cool the clocks for the device-resident configs)
    xt = hc.feeds[hc.x]
    hip.eval_many_with(hc.g, hc.roots, {hc.x: xt})
    t0 = time.perf_counter()
    for _ in range(2):
        hip.eval_many_with(hc.g, hc.roots, {hc.x: xt})
    host_ms = (time.perf_counter() - t0) * 1e3 / 2
    extra["cfg2_host_io"] = {"workload": "cfg 2 f32 via ku_eval_many (host feeds in, host tensors out)",
                             "ms_per_step": host_ms, "gbs": head["algo_bytes"] / (host_ms * 1e-3) / 1e9}
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_cfg2(xt)
        for key, fn in (("cfg2_bf16", lambda c: cpu_baseline_cfg2(c.feeds[c.x], "bf16")),
                        ("cfg1", lambda c: cpu_baseline_cfg1(c)), ("cfg3", lambda c: cpu_baseline_gemm(c, False)),
                        ("cfg3b", lambda c: cpu_baseline_gemm(c, True)), ("cfg4", cpu_baseline_attention),
                        ("cfg5", cpu_baseline_fp8)):
            if key in extra:
                extra[key]["cpu_baseline"] = fn(extra[key]["_cfg"])
    for v in extra.values():
        v.pop("_cfg", None)
    line = {
        "metric": "fused softmax+argmax HBM GB/s (cfg 2, f32 [8192,32000]); GEMM/attn TFLOP/s under configs",
        "value": round(head["value_gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: threefry2x32-seeded N(0, 3^2) logits generated on the device",
        "config": {"workload": head["workload"], "rows": 8192, "cols": 32000, "outputs": "softmax f32 + argmax i32",
                   "kernels": head["kernels"], "algo_bytes_per_step": head["algo_bytes"]},
        "roofline": head["roofline"],
        "cpu_baseline": cpu,
        "configs": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in extra.items()},
    }
    line["configs"]["cfg2_graph_replay"] = head["graph_replay"]
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
