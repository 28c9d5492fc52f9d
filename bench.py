"""kurumi_hip benchmark: the five headline configs on one MI355X, plus the CPU baseline.

The headline line (metric/value) is config 2 — row softmax over [8192, 32000] f32 built from
primitives (reduce_max, sub, exp, sum, div) followed by argmax -> int32 — as HBM GB/s of the
single fused kernel's algorithmic traffic. Every config runs as a device-resident plan
(inputs uploaded once, threefry-seeded synthetic data generated on the device), W untimed
launches, then K timed launches bracketed by stream synchronisation. Per-kernel durations
come from hipEvents recorded on the plan's own stream. The other configs are reported under
"configs" with their own roofline fractions; config "6" is the nn primitives around them
(rope, the SwiGLU gate, rmsnorm, the int4 decode GEMV).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs 1,2,3,4,5,6] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

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


def time_plan(plan, steps: int, warmup: int, use_graph: bool = False):
    """Warm up, then the timed region: `steps` back-to-back launches of the plan on its stream,
    bracketed by hipEvents on that stream (ku_hip_plan_time) and by a host clock around the call,
    which ends with the stream drained. Returns (wall ms per step, GPU ms of each plan step,
    step labels): the GPU time per launch comes from the timed region's events; a following
    run with events between the steps only splits it among the steps of a multi-kernel plan."""
    for _ in range(warmup):
        plan.launch(use_graph)
    plan.sync()
    t0 = time.perf_counter()
    gpu_ms = plan.time(steps, use_graph)
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    labels = plan.steps()
    if len(labels) == 1:
        return wall_ms, [gpu_ms], labels
    shares = plan.time_steps(max(steps, 5))
    tot = sum(shares)
    per_step = [s / tot * gpu_ms for s in shares] if tot > 0 else shares
    return wall_ms, per_step, labels


def measured_traffic(kernel: str):
    """HBM bytes per launch of a generated kernel, from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes (profiles/hbm_traffic.json, scaled by the copy-kernel calibration).
    Keyed by the kernel's name, which hashes its source: a changed kernel reads as null."""
    path = ROOT / "profiles" / "hbm_traffic.json"
    if not path.exists():
        return None
    rec = json.loads(path.read_text()).get("kernels", {}).get(kernel)
    return rec["traffic_bytes"] if rec else None


def roofline_hbm(bytes_per_launch: float, kernel_ms: float, kernel: str | None = None):
    gbs = bytes_per_launch / (kernel_ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(kernel) if kernel else None}


def roofline_mfma(flops: float, kernel_ms: float, peak_tflops: float):
    tf = flops / (kernel_ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": round(tf, 1), "peak": peak_tflops, "unit": "TFLOP/s",
            "frac": round(tf / peak_tflops, 4), "traffic": None}


# ---------------- config 2 (headline) ----------------

def softmax_graph(K, rows, cols, dt):
    g = K.Graph()
    x = g.input([rows, cols], dt)
    m = g.reduce_max(x, 1)
    e = g.exp(g.sub(x, g.expand(g.reshape(m, [rows, 1]), [rows, cols])))
    s = g.sum(e, 1)
    y = g.div(e, g.expand(g.reshape(s, [rows, 1]), [rows, cols]))
    a = g.cast(g.argmax(y, 1), K.DType.I32)
    return g, x, y, a


def bench_cfg2(hip, steps, warmup, dt_name="f32"):
    K = _ku()
    rows, cols = 8192, 32000
    dt = K.DType.F32 if dt_name == "f32" else K.DType.BF16
    xt = device_values(hip, scaled_randn(3.0), [rows, cols], 2024, dt)
    g, x, y, a = softmax_graph(K, rows, cols, dt)
    plan = hip.plan(g, [y, a], {x: xt})
    wall_ms, per_step, labels = time_plan(plan, steps, warmup)
    w = 4 if dt == K.DType.F32 else 2
    algo_bytes = rows * cols * w * 2 + rows * 4  # read x, write y, write int32 argmax
    kms = max(per_step)
    k = per_step.index(kms)
    return {
        "workload": f"softmax+argmax [{rows},{cols}] {dt_name} (decomposed primitives)",
        "ms_per_step": wall_ms, "kernels": labels, "kernel_ms": per_step, "dominant": labels[k],
        "algo_bytes": algo_bytes, "value_gbs": algo_bytes / (wall_ms * 1e-3) / 1e9,
        "roofline": roofline_hbm(algo_bytes, kms, labels[k]),
        "_graph": (g, x, y, a, xt),
    }


def cpu_baseline_cfg2(xt_full, rows_sample=256, cols=32000):
    """The oracle (single-threaded C++ restatement of kurumi's interpreter) on a row sample."""
    sys.path.insert(0, str(ROOT / "tests"))
    import kutest
    K = _ku()
    x_all = xt_full.numpy()
    xs = np.ascontiguousarray(x_all[:rows_sample])
    g, x, y, a = softmax_graph(K, rows_sample, cols, K.DType.F32)
    feeds = {x: K.Tensor.from_numpy(xs)}
    kutest.interpret(g, [y, a], feeds)  # warm-up
    reps, t0 = 0, time.perf_counter()
    while True:
        kutest.interpret(g, [y, a], feeds)
        reps += 1
        el = time.perf_counter() - t0
        if el > 8.0 or reps >= 20:
            break
    sec = el / reps
    algo_bytes = rows_sample * cols * 8 + rows_sample * 4
    return {"value": round(algo_bytes / sec / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{rows_sample} of 8192 rows x 32000 f32, decomposed softmax + argmax via the oracle "
                      f"interpreter, {reps} reps, {sec * 1e3:.1f} ms/rep, host nproc={os.cpu_count()}"}


# ---------------- other configs ----------------

def bench_cfg1(hip, steps, warmup):
    K = _ku()
    n = 4096
    plans = []
    # rotate 5 input sets (5 x 64 MiB > 256 MiB MALL) so the kernel streams from HBM
    for r in range(5):
        g = K.Graph()
        x = g.input([n, n], K.DType.F32)
        b = g.input([n], K.DType.F32)
        h = g.mul(g.relu(g.add(g.mul(x, x), g.broadcast_to(b, [n, n]))), g.scalar(x, 0.5))
        y = g.sum(h, 1)
        xt = device_values(hip, lambda gg, s, sd: gg.rand_range(s, sd, -1.0, 1.0), [n, n], 100 + r, K.DType.F32)
        bt = device_values(hip, lambda gg, s, sd: gg.rand_range(s, sd, -1.0, 1.0), [n], 200 + r, K.DType.F32)
        plans.append((hip.plan(g, [y], {x: xt, b: bt}), g))
    for _ in range(warmup):
        for p, _g in plans:
            p.launch()
    plans[0][0].sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        for p, _g in plans:
            p.launch()
    plans[0][0].sync()
    wall_ms = (time.perf_counter() - t0) * 1e3 / (steps * len(plans))
    algo_bytes = 4 * n * n + 4 * n + 4 * n
    return {"workload": "sum_lastaxis(relu(x*x+b)*0.5) [4096,4096] f32, 5 rotating input sets",
            "ms_per_step": wall_ms, "kernels": plans[0][0].steps(), "algo_bytes": algo_bytes,
            "roofline": roofline_hbm(algo_bytes, wall_ms, plans[0][0].steps()[0])}


def bench_gemm(hip, steps, warmup, batched=False):
    K = _ku()
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
    at = device_values(hip, scaled_randn(std), sa, 301, K.DType.BF16)
    bt = device_values(hip, scaled_randn(std), sb, 302, K.DType.BF16)
    plan = hip.plan(g, [c], {a: at, b: bt})
    wall_ms, per_step, labels = time_plan(plan, steps, warmup)
    kms = next(t for t, l in zip(per_step, labels) if l.startswith("gemm"))
    out = {"workload": ("batched [8,2048,128]@[8,128,2048]" if batched else "[4096,4096]@[4096,11008]") + " bf16",
           "ms_per_step": wall_ms, "kernels": labels, "kernel_ms": per_step, "flops": flops,
           "roofline": roofline_mfma(flops, kms, BF16_PEAK_TFLOPS)}
    if batched:
        byts = 2 * (8 * 2048 * 128 * 2) + 8 * 2048 * 2048 * 2
        out["roofline_hbm"] = roofline_hbm(byts, kms)
    return out


def bench_attention(hip, steps, warmup):
    K = _ku()
    B, H, S, D = 4, 32, 2048, 128
    g = K.Graph()
    q = g.input([B, H, S, D], K.DType.BF16)
    k = g.input([B, H, S, D], K.DType.BF16)
    v = g.input([B, H, S, D], K.DType.BF16)
    o = g.sdpa(q, k, v, True)
    feeds = {n: device_values(hip, lambda gg, s, sd: gg.randn(s, sd), [B, H, S, D], 400 + i, K.DType.BF16)
             for i, n in enumerate([q, k, v])}
    plan = hip.plan(g, [o], feeds)
    wall_ms, per_step, labels = time_plan(plan, steps, warmup)
    flops = 4 * B * H * S * S * D // 2
    return {"workload": "causal sdpa B4 H32 S2048 D128 bf16 (Op::Sdpa via g.sdpa)", "ms_per_step": wall_ms,
            "kernels": labels, "kernel_ms": per_step, "flops": flops,
            "roofline": roofline_mfma(flops, max(per_step), BF16_PEAK_TFLOPS)}


def bench_fp8(hip, steps, warmup):
    K = _ku()
    M, Kd, N = 2048, 4096, 11008
    wt = device_values(hip, scaled_randn(0.02), [N, Kd], 501, K.DType.F32)
    g = K.Graph()
    x = g.input([M, Kd], K.DType.BF16)
    w = g.constant_bytes(K.DType.F32, wt.data, [N, Kd])
    y0 = g.dot_general(x, g.cast(w, K.DType.BF16), [1], [1])
    y = K.amp_fp8(g, y0)
    xt = device_values(hip, lambda gg, s, sd: gg.randn(s, sd), [M, Kd], 502, K.DType.BF16)
    plan = hip.plan(g, [y], {x: xt})
    wall_ms, per_step, labels = time_plan(plan, steps, warmup)
    flops = 2 * M * N * Kd
    gemm_ms = next(t for t, l in zip(per_step, labels) if l.startswith("gemm"))
    return {"workload": "e4m3 linear X[2048,4096] W[11008,4096]^T per-row/per-tensor scales, bf16 out",
            "ms_per_step": wall_ms, "kernels": labels, "kernel_ms": per_step, "flops": flops,
            "roofline": roofline_mfma(flops, gemm_ms, FP8_PEAK_TFLOPS)}


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
    wall_ms, per_step, labels = time_plan(plan, steps, warmup)
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
        wall_ms, per_step, labels = time_plan(plan, steps, warmup)
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
        wall_ms, per_step, labels = time_plan(plan, steps, warmup)
        kms = sum(per_step) / layers
        algo = n * k // 2 + n * (k // grp) * 2 + m * k * 2 + m * n * 2  # packed weight, scales, act, out
        out[key] = {"workload": f"int4 (sym, group {grp}) {what} [{m},{k}] x [{n},{k}]^T bf16, "
                               f"{layers} layers' weights per plan", "ms_per_step": wall_ms / layers,
                    "kernels": labels[:1], "kernel_ms": per_step[:1], "algo_bytes": algo,
                    "roofline": roofline_hbm(algo, kms)}
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
    wall_ms, per_step, labels = time_plan(plan, steps, warmup)
    return {"workload": "copy 1 GiB f32 (y = -(-x))", "kernels": labels, "kernel_ms": per_step,
            "algo_bytes": 2 * 4 * n, "roofline": roofline_hbm(2 * 4 * n, max(per_step))}


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
    g, x, y, a, xt = head.pop("_graph")
    extra = {}
    if "2" in cfgs:
        b16 = bench_cfg2(hip, args.steps, args.warmup, "bf16")
        b16.pop("_graph")
        extra["cfg2_bf16"] = b16
    if "1" in cfgs:
        extra["cfg1"] = bench_cfg1(hip, args.steps, args.warmup)
    if "3" in cfgs:
        extra["cfg3"] = bench_gemm(hip, max(3, args.steps // 4), 1)
        extra["cfg3b"] = bench_gemm(hip, args.steps, args.warmup, batched=True)
    if "4" in cfgs:
        extra["cfg4"] = bench_attention(hip, max(3, args.steps // 4), 1)
    if "5" in cfgs:
        extra["cfg5"] = bench_fp8(hip, max(3, args.steps // 4), 1)
    if "6" in cfgs:
        extra.update(bench_nn(hip, args.steps, args.warmup))
        extra.update(bench_quant(hip, args.steps, args.warmup))
    if args.probe_copy:
        extra["copy_probe"] = bench_copy(hip, args.steps, args.warmup)
    # the same step through the host boundary (ku_eval_many with host feeds -> host results):
    # PCIe-inclusive rate, reported beside the device-resident value (last: the GPU idles while
    # the host copies, which would cool the clocks for the device-resident configs)
    hip.eval_many_with(g, [y, a], {x: xt})
    t0 = time.perf_counter()
    for _ in range(2):
        hip.eval_many_with(g, [y, a], {x: xt})
    host_ms = (time.perf_counter() - t0) * 1e3 / 2
    extra["cfg2_host_io"] = {"workload": "cfg 2 f32 via ku_eval_many (host feeds in, host tensors out)",
                             "ms_per_step": host_ms, "gbs": head["algo_bytes"] / (host_ms * 1e-3) / 1e9}
    cpu = None if args.no_cpu else cpu_baseline_cfg2(xt)
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
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
