"""Device plan replay (kurumi_core/src/realize/plan.rs:13-58; C ABI kurumi/src/capi/eval.rs:148-182).

`ku_plan_compile` builds a device plan once; `ku_plan_run` feeds it and replays it as one
hipGraph launch. Checked: replays with different feeds equal eager eval bit for bit and the
oracle within the dtype bars; multi-step plans (GEMM + fused region, attention, quantised
matmul, the e4m3 linear) replayed through hipGraphs several times, with other device work
between replays, equal their eager launches bit for bit; a process that used ku_plan_* exits
cleanly; and an equal graph rebuilt from the same KGPH blob reuses the plan and its uploaded
constants.
"""
import subprocess
import sys
import textwrap
from pathlib import Path

import numpy as np
import pytest

import bench
import kurumi_amd as K
from kurumi_amd import DType, Graph, Plan, Tensor
from kutest import assert_close, f32_to_bf16_bits, interpret, randn, to_f32

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parent.parent


def bf16_tensor(x: np.ndarray) -> Tensor:
    return Tensor(DType.BF16, x.shape, f32_to_bf16_bits(x).tobytes())


def test_ku_plan_run_replays_with_fresh_feeds(hip):
    print("ku_plan_compile / ku_plan_run softmax+argmax", flush=True)
    g, x, y, a = bench.softmax_graph(K, 64, 1000, DType.F32)
    for root in (y, a):
        plan = Plan(g, root)  # the process-default backend (ku_plan_compile)
        for seed in (1, 2, 3):
            feeds = {x: Tensor.from_numpy(randn([64, 1000], seed, 3.0))}
            got = plan.run(g, feeds)
            eager = hip.eval_with(g, root, feeds)
            np.testing.assert_array_equal(got.numpy(), eager.numpy())
            want = interpret(g, [root], feeds)[0]
            if root == a:
                np.testing.assert_array_equal(got.numpy(), want.numpy())
            else:
                assert_close(got.numpy(), want.numpy(), rtol=1e-4, atol=1e-30, what="plan replay vs oracle")


def test_ku_plan_on_a_backend_and_graph_checks(hip):
    g = Graph()
    xa = g.input([4, 256], DType.BF16)
    xb = g.input([256, 128], DType.BF16)
    c = g.rmsnorm(g.matmul(xa, xb), 1, 1e-6)
    plan = hip.compile(g, c)  # ku_hip_plan_compile_on
    for seed in (5, 6):
        feeds = {xa: bf16_tensor(randn([4, 256], seed)), xb: bf16_tensor(randn([256, 128], seed + 10))}
        np.testing.assert_array_equal(plan.run(g, feeds).numpy(), hip.eval_with(g, c, feeds).numpy())
    other = Graph()
    other.input([3], DType.F32)
    with pytest.raises(K.KuError, match="different graph"):
        plan.run(other, {})


def _multi_step_graphs():
    """(name, graph, roots, feeds builder) of plans with several steps of different kinds."""
    out = []
    g = Graph()  # GEMM, then a fused region reading its output
    a = g.input([96, 512], DType.BF16)
    b = g.input([512, 320], DType.BF16)
    y = g.softmax(g.matmul(a, b), 1)
    out.append(("gemm+softmax", g, [y, g.argmax(y, 1)],
                lambda s: {a: bf16_tensor(randn([96, 512], s, 0.1)), b: bf16_tensor(randn([512, 320], s + 1, 0.1))}))
    g2 = Graph()  # attention between two elementwise regions
    q, k, v = (g2.input([1, 2, 256, 128], DType.BF16) for _ in range(3))
    o = g2.sdpa_fused(g2.mul(q, g2.scalar(q, 0.5)), k, v, True)
    out.append(("attention", g2, [g2.sum(o, 3)],
                lambda s: {q: bf16_tensor(randn([1, 2, 256, 128], s)), k: bf16_tensor(randn([1, 2, 256, 128], s + 1)),
                           v: bf16_tensor(randn([1, 2, 256, 128], s + 2))}))
    g3 = Graph()  # int4 GEMV and fused MFMA quantised matmuls
    wv = np.random.default_rng(3).standard_normal((384, 512), dtype=np.float32)
    packed, scales, _ = K.quantize(wv, 4, 128, True)
    qw = g3.constant_bytes(DType.U8, packed.tobytes(), packed.shape)
    sc = g3.constant_bytes(DType.F16, scales.tobytes(), scales.shape)
    x1 = g3.input([1, 512], DType.BF16)
    x32 = g3.input([32, 512], DType.BF16)
    out.append(("quant", g3, [g3.quant_matmul(x1, qw, sc, None, 4, 128), g3.quant_matmul(x32, qw, sc, None, 4, 128)],
                lambda s: {x1: bf16_tensor(randn([1, 512], s)), x32: bf16_tensor(randn([32, 512], s + 1))}))
    w8 = (np.random.default_rng(4).standard_normal((256, 512), dtype=np.float32) * 0.02).astype(np.float32)
    g4, x4, y4 = bench.fp8_graph(K, [128, 512], w8.tobytes(), [256, 512])
    out.append(("e4m3 linear", g4, [y4], lambda s: {x4: bf16_tensor(randn([128, 512], s))}))
    return out


@pytest.mark.parametrize("case", range(4))
def test_hipgraph_replay_equals_eager_launch(hip, case):
    name, g, roots, mk = _multi_step_graphs()[case]
    print(f"hipGraph replay {name}", flush=True)
    plan = hip.plan(g, roots, mk(100))
    assert len(plan.steps()) >= 2, plan.steps()
    for rep, seed in enumerate((100, 100, 101, 102)):
        feeds = mk(seed)
        for n, t in feeds.items():
            plan.feed(n, t)
        plan.launch(use_graph=False)
        eager = [plan.output(i) for i in range(len(roots))]
        # other device work between the eager launch and the replay
        hip.eval_with(g, roots[0], feeds)
        plan.launch(use_graph=True)
        replay = [plan.output(i) for i in range(len(roots))]
        for i, (e, r) in enumerate(zip(eager, replay)):
            np.testing.assert_array_equal(r.numpy(), e.numpy(), err_msg=f"{name} replay {rep} output {i}")
        want = interpret(g, roots, feeds)
        for i, (r, w) in enumerate(zip(replay, want)):
            if r.dtype in (DType.I32, DType.I64):
                np.testing.assert_array_equal(r.numpy(), w.numpy())
            else:
                tol = 3e-2 if name == "e4m3 linear" else 1e-2
                wf = to_f32(w)
                assert_close(to_f32(r), wf, rtol=tol, atol=tol * np.abs(wf).max(), what=f"{name} output {i} vs oracle")


def test_process_using_ku_plan_exits_cleanly():
    """The process-default backend behind ku_plan_compile outlives static destruction."""
    code = textwrap.dedent(f"""
        import sys
        sys.path.insert(0, {str(ROOT)!r})
        import numpy as np
        import kurumi_amd as K
        g = K.Graph()
        x = g.input([8, 300], K.DType.F32)
        y = g.softmax(x, 1)
        p = K.Plan(g, y)
        t = p.run(g, {{x: K.Tensor.from_numpy(np.ones((8, 300), np.float32))}})
        assert np.allclose(t.numpy(), 1.0 / 300)
        print("ran", flush=True)
    """)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "ran" in r.stdout, (r.returncode, r.stdout, r.stderr[-2000:])


def test_plans_outlive_the_backend_handle_they_were_built_on():
    """ku_backend_free before ku_plan_free / ku_hip_plan_free: the plans keep the backend (its
    stream, pools and constant cache) alive, run correctly after the handle is gone, and the
    process exits cleanly once the last plan is freed."""
    code = textwrap.dedent(f"""
        import ctypes as C, sys
        sys.path.insert(0, {str(ROOT)!r})
        import numpy as np
        import kurumi_amd as K
        L = K.lib()
        g = K.Graph()
        x = g.input([16, 300], K.DType.F32)
        w = g.constant(np.linspace(-1, 1, 300 * 64, dtype=np.float32).reshape(300, 64))
        y = g.softmax(g.matmul(x, w), 1)
        xv = np.random.default_rng(3).standard_normal((16, 300)).astype(np.float32)
        feeds = K.Feeds({{x: K.Tensor.from_numpy(xv)}})
        ref = K.HipBackend()
        want = ref.eval_with(g, y, {{x: K.Tensor.from_numpy(xv)}}).numpy()
        b = L.ku_backend_new(2)
        assert b
        p = L.ku_hip_plan_compile_on(b, g.h, y)
        roots = (C.c_uint32 * 1)(y)
        hp = L.ku_hip_plan_new(g.h, roots, 1, b, feeds.h)
        assert p and hp
        L.ku_backend_free(b)
        print("backend handle freed", flush=True)
        t = K.Tensor._from_handle(L.ku_plan_run(p, g.h, feeds.h))
        np.testing.assert_array_equal(t.numpy(), want)
        assert L.ku_hip_plan_launch(hp, 1) == 0 and L.ku_hip_plan_sync(hp) == 0
        np.testing.assert_array_equal(K.Tensor._from_handle(L.ku_hip_plan_output(hp, 0)).numpy(), want)
        L.ku_plan_free(p)
        L.ku_hip_plan_free(hp)
        print("ran", flush=True)
    """)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "ran" in r.stdout, (r.returncode, r.stdout, r.stderr[-2000:])


def test_equal_graphs_from_one_blob_share_plan_and_constants(hip):
    """The KGPH seam decodes a fresh graph per call: the second decode finds the first's plan and
    weights by content (no new plan, no new constant upload), and results stay identical."""
    print("content-keyed plan reuse", flush=True)
    g = Graph()
    x = g.input([16, 1024], DType.F32)
    w = g.constant(np.random.default_rng(9).standard_normal((1024, 512)).astype(np.float32))
    y = g.sum(g.relu(g.matmul(x, w)), 1)
    blob = K.serialize_reachable(g, [y], [K.InputBinding(x, K.InputRole.Runtime, "x")])
    feeds_v = Tensor.from_numpy(randn([16, 1024], 77))
    r1 = K.deserialize_graph(blob)
    first = hip.eval_with(r1.graph, r1.outputs[0], {r1.inputs[0].node: feeds_v})
    before = hip.profile()
    r2 = K.deserialize_graph(blob)
    second = hip.eval_with(r2.graph, r2.outputs[0], {r2.inputs[0].node: feeds_v})
    after = hip.profile()
    np.testing.assert_array_equal(first.numpy(), second.numpy())
    assert after["plans_built"] == before["plans_built"], (before, after)
    assert after["const_uploads"] == before["const_uploads"], (before, after)
    # a different weight is a different graph
    g3 = Graph()
    x3 = g3.input([16, 1024], DType.F32)
    w3 = g3.constant(np.random.default_rng(10).standard_normal((1024, 512)).astype(np.float32))
    y3 = g3.sum(g3.relu(g3.matmul(x3, w3)), 1)
    third = hip.eval_with(g3, y3, {x3: feeds_v})
    assert hip.profile()["plans_built"] == after["plans_built"] + 1
    assert not np.array_equal(third.numpy(), first.numpy())


def test_a_plan_that_runs_out_of_device_memory_gives_its_buffers_back():
    """A device plan whose buffers do not fit (102 GB + 256 GB outputs on a 288 GB GPU) fails with
    an error naming the failed allocation, and the backend gets back what that plan had already
    allocated: a 205 GB plan on the same backend then fits (it would not beside a leaked 102 GB).
    Run in a child process so nothing it holds can crowd the other tests."""
    code = textwrap.dedent(f"""
        import sys
        sys.path.insert(0, {str(ROOT)!r})
        import numpy as np
        import kurumi_amd as K
        be = K.HipBackend()

        def big(rows_list):
            g = K.Graph()
            x = g.input([1, 1024], K.DType.F32)
            ys = [g.expand(g.mul(x, g.scalar(x, float(i + 2))), [r, 1024]) for i, r in enumerate(rows_list)]
            return g, x, ys

        g, x, ys = big([25_000_000, 62_500_000])
        feeds = {{x: K.Tensor.from_numpy(np.ones((1, 1024), np.float32))}}
        try:
            K.HipPlan(be, g, ys, feeds)
            raise SystemExit("the 358 GB plan was built")
        except K.KuError as e:
            msg = str(e)
        assert "hipMalloc" in msg or "memory" in msg.lower(), msg
        print("failed as expected:", msg.splitlines()[0][:160], flush=True)
        g2, x2, ys2 = big([50_000_000])
        p = K.HipPlan(be, g2, ys2, {{x2: K.Tensor.from_numpy(np.ones((1, 1024), np.float32))}})
        del p
        print("ran", flush=True)
    """)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "ran" in r.stdout, (r.returncode, r.stdout, r.stderr[-2000:])
