"""Device parity of Op::QuantMatmul (the fused dequant GEMV for M <= 8, dequantize + GEMM above).

Against the oracle (dequantize, f32 contraction, one rounding to act's dtype) and against an
f64 product of numpy-dequantized weights: f32 <= 1e-5 normwise; bf16 / f16 <= 1e-2 (the GEMM
path also rounds each dequantized weight to act's dtype once).
"""
import numpy as np
import pytest

import kurumi_amd as K
from kurumi_amd import DType, Graph, Tensor
from kutest import assert_close, interpret, rel_err, to_f32
from test_quant import dequant

pytestmark = pytest.mark.gpu


def build(m, n, k, bits, group, sym, act_dt, seed):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((n, k)).astype(np.float32)
    act = rng.standard_normal((m, k)).astype(np.float32)
    p, s, mn = K.quantize(w, bits, group, sym)
    g = Graph()
    x = g.input([m, k], act_dt)
    qw = g.constant_bytes(DType.U8, p.tobytes(), p.shape)
    sc = g.constant_bytes(DType.F16, s.tobytes(), s.shape)
    mnn = None if mn is None else g.constant_bytes(DType.F16, mn.tobytes(), mn.shape)
    y = g.quant_matmul(x, qw, sc, mnn, bits, group)
    if act_dt == DType.F32:
        xt = Tensor.from_numpy(act)
    else:
        xt = interpret(*(lambda gg: (gg, [gg.cast(gg.constant(act), act_dt)]))(Graph()))[0]
    truth = to_f32(xt).astype(np.float64) @ dequant(p, s, mn, k, bits, group).astype(np.float64).T
    return g, x, y, xt, truth


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 9, 17, 64])
@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("sym", [True, False])
@pytest.mark.parametrize("act_dt", [DType.F32, DType.BF16])
def test_quant_matmul_matches_oracle(hip, m, bits, sym, act_dt):
    print(f"quant m={m} bits={bits} sym={sym} {act_dt.name}", flush=True)
    g, x, y, xt, truth = build(m, 96, 256, bits, 64, sym, act_dt, 100 + m + bits)
    feeds = {x: xt}
    got = to_f32(hip.eval_with(g, y, feeds))
    want = to_f32(interpret(g, [y], feeds)[0])
    tol = 1e-5 if act_dt == DType.F32 else 1e-2
    assert rel_err(got, truth) <= tol, rel_err(got, truth)
    assert_close(got, want, rtol=tol, atol=tol * np.abs(want).max(), what="quant vs oracle")


@pytest.mark.parametrize("k,group,bits", [(40, 8, 4), (24, 24, 8), (64, 16, 2), (96, 96, 4)])
def test_quant_gemv_odd_rows_and_groups(hip, k, group, bits):
    """Rows that are not whole 16-byte chunks, and groups smaller than a chunk's fields."""
    print(f"quant odd k={k} g={group} bits={bits}", flush=True)
    for m in (1, 3, 7):
        g, x, y, xt, truth = build(m, 37, k, bits, group, False, DType.F32, 7 + k)
        got = hip.eval_with(g, y, {x: xt}).numpy()
        assert rel_err(got, truth) <= 1e-5


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("sym", [True, False])
def test_quant_f16_act(hip, bits, sym):
    """f16 act (the v_dot2_f32_f16 path for 2- and 4-bit fields, whose 1024 + u trick has the
    largest cancellation), M = 1 .. 3."""
    for m in (1, 3):
        g, x, y, xt, truth = build(m, 64, 256, bits, 32, sym, DType.F16, 9 + bits + m)
        got = to_f32(hip.eval_with(g, y, {x: xt}))
        assert rel_err(got, truth) <= 1e-2
        want = to_f32(interpret(g, [y], {x: xt})[0])
        assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what="f16 quant vs oracle")


def test_quant_decode_full_size(hip):
    """The decode shape: one token through an int4 (group 128) [11008, 4096] projection, bf16."""
    print("quant decode 1x4096 -> 11008", flush=True)
    g, x, y, xt, truth = build(1, 11008, 4096, 4, 128, True, DType.BF16, 11)
    got = to_f32(hip.eval_with(g, y, {x: xt}))
    assert rel_err(got, truth) <= 1e-2
    assert_close(got, truth, rtol=1e-2, atol=1e-2 * np.abs(truth).max(), what="decode")


@pytest.mark.parametrize("m", [9, 32, 33, 64])
@pytest.mark.parametrize("sym", [True, False])
@pytest.mark.parametrize("act_dt", [DType.BF16, DType.F16])
@pytest.mark.parametrize("group", [64, 128, 256])
def test_quant_mfma_path_matches_oracle(hip, m, sym, act_dt, group):
    """The fused dequant MFMA kernel (int4, 9 <= M <= 64): row counts that cut the 32-row weight
    tiles (100) and the 32-row act tiles (9, 33), every group size it takes."""
    print(f"quant mfma m={m} sym={sym} {act_dt.name} g={group}", flush=True)
    g, x, y, xt, truth = build(m, 100, 512, 4, group, sym, act_dt, 300 + m + group)
    steps = [l for l in g.codegen([y]).splitlines() if l.startswith("// step ")]
    assert any("quant_mfma" in st for st in steps), steps
    got = to_f32(hip.eval_with(g, y, {x: xt}))
    assert rel_err(got, truth) <= 1e-2, rel_err(got, truth)
    want = to_f32(interpret(g, [y], {x: xt})[0])
    assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what="quant mfma vs oracle")


@pytest.mark.parametrize("m,n,k,group,sym", [(17, 100, 512, 128, True), (32, 300, 1024, 256, False),
                                             (40, 100, 2048, 128, True), (64, 70, 512, 128, False)])
def test_quant_mfma_weight_input_matches_constant(hip, m, n, k, group, sym):
    """The fused MFMA kernel reads a constant weight from the planner's lane-ordered copy and a
    weight fed as an input as it is (row-major): the same products and sums in the same order, so
    the two are bit-identical, and both match the oracle. Rows (70, 100, 300) cut the 32-row
    tiles; M = 40 and 64 take the 64-row act tile."""
    print(f"quant mfma weight input m={m} n={n} k={k} g={group} sym={sym}", flush=True)
    gc, xc, yc, xt, truth = build(m, n, k, 4, group, sym, DType.BF16, 900 + m)
    steps = [l for l in gc.codegen([yc]).splitlines() if l.startswith("// step ")]
    assert any("quant_mfma" in st for st in steps), steps
    const = hip.eval_with(gc, yc, {xc: xt})
    rng = np.random.default_rng(900 + m)
    w = rng.standard_normal((n, k)).astype(np.float32)  # the weights build() quantised
    p, s, mn = K.quantize(w, 4, group, sym)
    g = Graph()
    x = g.input([m, k], DType.BF16)
    qw = g.input(list(p.shape), DType.U8)
    sc = g.input(list(s.shape), DType.F16)
    mnn = None if mn is None else g.input(list(mn.shape), DType.F16)
    y = g.quant_matmul(x, qw, sc, mnn, 4, group)
    feeds = {x: xt, qw: Tensor.from_numpy(p), sc: Tensor.from_numpy(s, DType.F16)}
    if mnn is not None:
        feeds[mnn] = Tensor.from_numpy(mn, DType.F16)
    fed = hip.eval_with(g, y, feeds)
    assert bytes(fed.data) == bytes(const.data), "weight input and constant weight differ"
    got = to_f32(fed)
    assert rel_err(got, truth) <= 1e-2, rel_err(got, truth)
    want = to_f32(interpret(g, [y], feeds)[0])
    assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what="quant mfma (weight input) vs oracle")


def test_quant_constant_weight_shared_by_plans(hip):
    """One constant int4 weight in several plans on one backend: the batched path's plans (M = 32
    and M = 17) read the lane-ordered copy the constant's cache entry holds, made by the first of
    them; the decode plan (M = 1) reads the packed bytes themselves. Dropping the plan that made
    the copy leaves it to the others (it lives as long as the constant), so every plan, launched
    again afterwards, still matches the oracle."""
    import gc
    n, k, group = 300, 1024, 128
    rng = np.random.default_rng(41)
    w = rng.standard_normal((n, k)).astype(np.float32)
    p, s, _ = K.quantize(w, 4, group, True)
    plans = {}
    for m in (32, 17, 1):
        g = Graph()
        x = g.input([m, k], DType.BF16)
        qw = g.constant_bytes(DType.U8, p.tobytes(), p.shape)
        sc = g.constant_bytes(DType.F16, s.tobytes(), s.shape)
        y = g.quant_matmul(x, qw, sc, None, 4, group)
        act = rng.standard_normal((m, k)).astype(np.float32)
        xt = interpret(*(lambda gg: (gg, [gg.cast(gg.constant(act), DType.BF16)]))(Graph()))[0]
        plan = hip.plan(g, [y], {x: xt})
        assert plan.steps()[0].startswith("quant_mfma" if m > 8 else "quant_gemv"), plan.steps()
        plans[m] = (plan, g, x, y, xt)

    def check(m):
        plan, g, x, y, xt = plans[m]
        plan.launch()
        plan.sync()
        got = to_f32(plan.output(0))
        want = to_f32(interpret(g, [y], {x: xt})[0])
        assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what=f"shared weight m={m}")

    for m in (32, 17, 1):
        check(m)
    del plans[32]  # the plan whose build made the lane-ordered copy
    gc.collect()
    for m in (17, 1):
        check(m)


@pytest.mark.parametrize("sym", [True, False])
@pytest.mark.parametrize("m,n", [(17, 99), (40, 35)])
def test_quant_mfma_odd_group_count_and_rows(hip, m, n, sym):
    """The fused MFMA kernel with an odd number of scale groups per row (k / group = 3) and an odd
    row count in the last work-group's tile: the table's last scale (and min) shares a dword
    with the row past N, and must still be read."""
    print(f"quant mfma odd ng m={m} n={n} sym={sym}", flush=True)
    g, x, y, xt, truth = build(m, n, 384, 4, 128, sym, DType.BF16, 900 + m + n)
    plan = hip.plan(g, [y], {x: xt})
    assert plan.steps()[0].startswith("quant_mfma"), plan.steps()
    got = to_f32(hip.eval_with(g, y, {x: xt}))
    want = to_f32(interpret(g, [y], {x: xt})[0])
    assert rel_err(got, truth) <= 1e-2, rel_err(got, truth)
    assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what="odd-ng quant mfma vs oracle")
    # the last row's last group alone: its scale must not read as 0
    assert np.abs(got[:, -1] - want[:, -1]).max() <= 1e-2 * np.abs(want).max()


def test_quant_constant_weight_read_at_two_shapes(hip):
    """One packed int4 constant read as [256, 1024] and, reshaped, as [512, 512] (each packed row
    split in two, its scale row with it). The constant's cache entry keeps one lane-ordered copy
    per shape, so neither read loses its copy to the other: within one plan, and across two plans
    that share the constant by content, every output matches the oracle, also when the first
    plan is launched again after the second was built."""
    n, k, group, m = 256, 1024, 128, 32
    rng = np.random.default_rng(43)
    w = rng.standard_normal((n, k)).astype(np.float32)
    p, s, _ = K.quantize(w, 4, group, True)

    def graph(shapes):
        g = Graph()
        qw = g.constant_bytes(DType.U8, p.tobytes(), p.shape)
        sc = g.constant_bytes(DType.F16, s.tobytes(), s.shape)
        ins, outs = [], []
        for rows in shapes:  # rows of the weight it is read as: n or 2n
            kk = n * k // rows
            x = g.input([m, kk], DType.BF16)
            q = qw if rows == n else g.reshape(qw, [rows, kk // 2])
            c = sc if rows == n else g.reshape(sc, [rows, kk // group])
            ins.append(x)
            outs.append(g.quant_matmul(x, q, c, None, 4, group))
        return g, ins, outs

    acts = {rows: interpret(*(lambda gg: (gg, [gg.cast(gg.constant(
        rng.standard_normal((m, n * k // rows)).astype(np.float32)), DType.BF16)]))(Graph()))[0] for rows in (n, 2 * n)}

    def check(plan, g, ins, outs, shapes, what):
        plan.launch()
        plan.sync()
        feeds = {x: acts[rows] for x, rows in zip(ins, shapes)}
        wants = interpret(g, outs, feeds)
        for i, rows in enumerate(shapes):
            got, want = to_f32(plan.output(i)), to_f32(wants[i])
            assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what=f"{what} rows={rows}")

    # one plan, both shapes
    g, ins, outs = graph([n, 2 * n])
    plan = hip.plan(g, outs, {ins[0]: acts[n], ins[1]: acts[2 * n]})
    assert all(st.startswith("quant_mfma") for st in plan.steps()), plan.steps()
    check(plan, g, ins, outs, [n, 2 * n], "one plan")
    # two plans sharing the constant
    ga, ia, oa = graph([n])
    pa = hip.plan(ga, oa, {ia[0]: acts[n]})
    gb, ib, ob = graph([2 * n])
    pb = hip.plan(gb, ob, {ib[0]: acts[2 * n]})
    check(pb, gb, ib, ob, [2 * n], "second plan")
    check(pa, ga, ia, oa, [n], "first plan after the second")
    check(plan, g, ins, outs, [n, 2 * n], "one plan again")


def test_quant_mfma_batched_decode_size(hip):
    """A batch of 32 tokens through the int4 (group 128) [11008, 4096] projection."""
    print("quant mfma 32x4096 -> 11008", flush=True)
    g, x, y, xt, truth = build(32, 11008, 4096, 4, 128, True, DType.BF16, 12)
    got = to_f32(hip.eval_with(g, y, {x: xt}))
    assert rel_err(got, truth) <= 1e-2
    assert_close(got, truth, rtol=1e-2, atol=1e-2 * np.abs(truth).max(), what="batched decode")


@pytest.mark.parametrize("m,k,group,sym,act_dt", [(33, 2048, 64, False, DType.F16), (20, 4096, 256, True, DType.BF16),
                                                  (64, 1024, 128, False, DType.BF16)])
def test_quant_mfma_long_k_matches_oracle(hip, m, k, group, sym, act_dt):
    """Longer K: every wave of the MFMA kernel takes several sub-groups (the one-ahead prefetch
    runs), groups of 64 (one block per sub-group) and 256 (two sub-groups per scale)."""
    print(f"quant mfma long k m={m} k={k} g={group} sym={sym} {act_dt.name}", flush=True)
    g, x, y, xt, truth = build(m, 100, k, 4, group, sym, act_dt, 500 + m + k)
    got = to_f32(hip.eval_with(g, y, {x: xt}))
    assert rel_err(got, truth) <= 1e-2, rel_err(got, truth)
    if m * k <= 33 * 2048:
        want = to_f32(interpret(g, [y], {x: xt})[0])
        assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what="long-K quant mfma vs oracle")
