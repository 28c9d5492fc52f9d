"""Full-size parity of the exact plans bench.py times.

Each test builds its config through bench.py's own `make_*` function (same graph, same shapes,
same device-generated inputs), so the kernel variants checked here are the ones the bench
reports; the plan's step labels are asserted so a change of variant shows. Rows (and heads)
are independent in every config, so the oracle checks a stated sample of them at full size;
everything else is checked over the whole output against f64 or a size-independent property.

Bars: argmax / integer outputs bit-exact; f32 <= 1e-5 relative (against f64; the oracle's own
sequential f32 folds are bounded at 1e-4); bf16 <= 1e-2; e4m3 linear <= 3e-2 against the
dequantised-f64 product sx * sw[n] * sum_k f64(Xq[m,k]) * f64(Wq[n,k]).
"""
import numpy as np
import pytest

import bench
import kurumi_amd as K
from kurumi_amd import DType, Tensor
from kutest import (assert_close, bf16_bits_to_f32, bf16_ulp, cast_bits, f32_to_bf16_bits, interpret, rel_err, to_f32)

pytestmark = pytest.mark.gpu


def row_sample(n: int, edge: int, mid: int, seed: int) -> np.ndarray:
    """The first and last `edge` rows plus `mid` random rows between them, sorted."""
    rng = np.random.default_rng(seed)
    inner = rng.choice(np.arange(edge, n - edge), size=mid, replace=False)
    return np.unique(np.concatenate([np.arange(edge), inner, np.arange(n - edge, n)]))


def softmax_f64_rows(x: np.ndarray) -> np.ndarray:
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


# ---------------- config 2 ----------------

@pytest.mark.parametrize("dt_name", ["f32", "bf16"])
def test_cfg2_bench_plan_full_size(hip, dt_name):
    print(f"cfg2 bench plan {dt_name} [8192,32000]", flush=True)
    c = bench.make_cfg2(hip, dt_name)
    labels = c.plan.steps()
    assert len(labels) == 1 and labels[0].startswith("ku_line_8192x32000_"), labels
    c.plan.launch()
    y_t, a_t = c.plan.output(0), c.plan.output(1)
    a = a_t.numpy()
    assert a_t.dtype == DType.I32 and a.shape == (c.rows,)
    xbits = c.feeds[c.x].numpy()
    x = xbits if dt_name == "f32" else bf16_bits_to_f32(xbits)
    y = to_f32(y_t)
    # every row: the argmax epilogue is the first index of the stored row's maximum
    np.testing.assert_array_equal(a, np.argmax(y, axis=1))
    # softmax is monotone: the input's maximum lands on a maximal output
    assert (y[np.arange(c.rows), np.argmax(x, axis=1)] == y.max(axis=1)).all()
    if dt_name == "f32":
        for r0 in range(0, c.rows, 1024):  # every row against f64, in chunks
            assert_close(y[r0:r0 + 1024], softmax_f64_rows(x[r0:r0 + 1024]), rtol=1e-5, atol=1e-30,
                         what=f"softmax f32 rows {r0}.. vs f64")
    else:
        s = y.astype(np.float64).sum(axis=1)
        assert np.abs(s - 1.0).max() <= 1e-2, np.abs(s - 1.0).max()
    # the oracle on a row sample (first/last 128 rows + 256 random): argmax bit-exact
    rows = row_sample(c.rows, 128, 256, 5)
    g, xs, ys, as_ = bench.softmax_graph(K, len(rows), c.cols, c.dt)
    feeds = {xs: Tensor(c.dt, [len(rows), c.cols], np.ascontiguousarray(xbits[rows]).tobytes())}
    wy, wa = interpret(g, [ys, as_], feeds)
    np.testing.assert_array_equal(a[rows], wa.numpy())
    if dt_name == "f32":
        assert_close(y[rows], to_f32(wy), rtol=1e-4, atol=1e-30, what="softmax f32 vs oracle")
    else:
        want = to_f32(wy)  # elementwise: 1e-2 of each element plus one bf16 step at its magnitude
        assert_close(y[rows], want, rtol=1e-2, atol=bf16_ulp(want), what="softmax bf16 vs oracle")


# ---------------- config 1 ----------------

def test_cfg1_bench_plan_full_size(hip):
    print("cfg1 bench plan [4096,4096]", flush=True)
    c = bench.make_cfg1(hip, 0)
    labels = c.plan.steps()
    assert len(labels) == 1 and labels[0].startswith("ku_line_4096x4096_"), labels
    c.plan.launch()
    got = c.plan.output(0).numpy()
    xv, bv = c.feeds[c.x].numpy(), c.feeds[c.b].numpy()
    h = np.maximum(xv * xv + bv[None, :], np.float32(0)) * np.float32(0.5)
    truth = h.astype(np.float64).sum(axis=1)
    assert_close(got, truth, rtol=1e-5, atol=1e-5 * np.abs(truth).max(), what="cfg1 vs f64")
    want = interpret(c.g, c.roots, c.feeds)[0].numpy()
    assert_close(got, want, rtol=2e-5, atol=2e-5 * np.abs(want).max(), what="cfg1 vs oracle")


# ---------------- config 3 ----------------

def bf16_f64(t: Tensor) -> np.ndarray:
    return bf16_bits_to_f32(t.numpy()).astype(np.float64)


def test_cfg3_bench_plan_full_size(hip):
    print("cfg3 bench plan [4096,4096]@[4096,11008]", flush=True)
    c = bench.make_gemm(hip, batched=False)
    assert c.plan.steps() == ["gemm_mfma_bf16_nn_256x256 b1 m4096 n11008 k4096"]
    c.plan.launch()
    got = to_f32(c.plan.output(0))
    A, B = bf16_f64(c.feeds[c.a]), bf16_f64(c.feeds[c.b])
    # the first and last 256-row tile, 256 random rows between; every output column
    rows = row_sample(4096, 256, 256, 3)
    truth = A[rows] @ B
    assert rel_err(got[rows], truth) <= 1e-2
    assert_close(got[rows], truth, rtol=1e-2, atol=1e-2 * np.abs(truth).max(), what="cfg3 vs f64")
    # the oracle (f32 GEMM of the bf16 inputs, rounded once to bf16) on 16 of those rows: both
    # round an f32 sum of the same products, so they agree to a bf16 step except where the f32
    # sums' different orders straddle a rounding boundary near zero
    orows = np.concatenate([rows[:4], rows[len(rows) // 2 - 4:len(rows) // 2 + 4], rows[-4:]])
    g = K.Graph()
    a = g.input([len(orows), 4096], DType.BF16)
    b = g.input([4096, 11008], DType.BF16)
    y = g.matmul(a, b)
    abits = np.ascontiguousarray(c.feeds[c.a].numpy()[orows])
    want = to_f32(interpret(g, [y], {a: Tensor(DType.BF16, [len(orows), 4096], abits.tobytes()), b: c.feeds[c.b]})[0])
    assert_close(got[orows], want, rtol=1e-2, atol=bf16_ulp(want) + 1e-4 * np.abs(want).max(), what="cfg3 vs oracle")


def test_cfg3b_bench_plan_full_size(hip):
    print("cfg3b bench plan [8,2048,128]@[8,128,2048]", flush=True)
    c = bench.make_gemm(hip, batched=True)
    assert c.plan.steps() == ["gemm_mfma_bf16_nn_128x128_persistent b8 m2048 n2048 k128"]
    c.plan.launch()
    got = to_f32(c.plan.output(0))
    truth = np.matmul(bf16_f64(c.feeds[c.a]), bf16_f64(c.feeds[c.b]))
    assert rel_err(got, truth) <= 1e-2
    assert_close(got, truth, rtol=1e-2, atol=1e-2 * np.abs(truth).max(), what="cfg3b vs f64")
    # the oracle on batch 0's first and last 64 rows
    g = K.Graph()
    a = g.input([1, 128, 128], DType.BF16)
    b = g.input([1, 128, 2048], DType.BF16)
    y = g.dot_general(a, b, [2], [1], [0], [0])
    abits = c.feeds[c.a].numpy()[:1, np.r_[0:64, 2048 - 64:2048]]
    feeds = {a: Tensor(DType.BF16, [1, 128, 128], np.ascontiguousarray(abits).tobytes()),
             b: Tensor(DType.BF16, [1, 128, 2048], np.ascontiguousarray(c.feeds[c.b].numpy()[:1]).tobytes())}
    want = to_f32(interpret(g, [y], feeds)[0])
    assert_close(got[:1, np.r_[0:64, 2048 - 64:2048]], want, rtol=1e-2, atol=1e-2 * np.abs(want).max(),
                 what="cfg3b vs oracle")


# ---------------- config 4 ----------------

def test_cfg4_bench_plan_heads_match_oracle(hip):
    print("cfg4 bench plan [4,32,2048,128] causal", flush=True)
    c = bench.make_attention(hip)
    labels = c.plan.steps()
    assert len(labels) == 1 and labels[0].startswith("attn_mfma") and "causal" in labels[0], labels
    c.plan.launch()
    got = to_f32(c.plan.output(0))
    assert np.isfinite(got).all()
    S, D = 2048, 128
    for bi, hi in ((0, 0), (3, 31), (2, 17)):  # first, last and one middle head
        g = K.Graph()
        q, k, v = (g.input([1, 1, S, D], DType.BF16) for _ in range(3))
        o = g.sdpa_fused(q, k, v, True)
        feeds = {n: Tensor(DType.BF16, [1, 1, S, D], np.ascontiguousarray(c.feeds[src].numpy()[bi, hi]).tobytes())
                 for n, src in ((q, c.q), (k, c.k), (v, c.v))}
        want = to_f32(interpret(g, [o], feeds)[0])[0, 0]
        assert rel_err(got[bi, hi], want) <= 1e-2
        assert_close(got[bi, hi], want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what=f"cfg4 head {bi},{hi}")


# ---------------- config 5 ----------------

def e4m3_f64(x_f32: np.ndarray) -> np.ndarray:
    """Round f32 values to e4m3 (the oracle's bit-exact cast) and widen them to f64."""
    q = cast_bits(np.ascontiguousarray(x_f32, dtype=np.float32).reshape(-1), DType.F32, DType.F8E4M3)
    return cast_bits(q, DType.F8E4M3, DType.F64).view(np.float64).reshape(x_f32.shape)


def dequant_f64_linear(x_bf16_bits: np.ndarray, w_f32: np.ndarray) -> np.ndarray:
    """cfg 5's stated oracle: sx * sw[n] * sum_k f64(Xq[m,k]) * f64(Wq[n,k]) with
    sw[n] = max_k |W[n,k]| / 448 and Wq = e4m3(W / sw[n]) per weight row, and the per-tensor
    sx = max |X| * (1/448), Xq = e4m3(X * (1/sx)), all scale arithmetic in f32."""
    x = bf16_bits_to_f32(x_bf16_bits)
    sw = (np.abs(w_f32).max(axis=1) / np.float32(448.0)).astype(np.float32)
    sw[~(sw > 0)] = 1.0
    wq = e4m3_f64(w_f32 / sw[:, None])
    sx = np.float32(np.abs(x).max()) * np.float32(1.0 / 448.0)
    xq = e4m3_f64(x * (np.float32(1.0) / sx))
    return (xq @ wq.T) * np.float64(sx) * sw.astype(np.float64)[None, :]


def test_cfg5_bench_plan_matches_dequantised_f64(hip):
    print("cfg5 bench plan [2048,4096] x [11008,4096]^T e4m3", flush=True)
    c = bench.make_fp8(hip)
    labels = c.plan.steps()
    assert labels[-1] == "gemm_mfma_e4m3_nt_192x256 b1 m2048 n11008 k4096", labels
    c.plan.launch()
    got = to_f32(c.plan.output(0))
    w = np.frombuffer(c.w.data, np.float32).reshape(c.N, c.K)
    truth = dequant_f64_linear(c.feeds[c.x].numpy(), w)
    assert rel_err(got, truth) <= 3e-2
    assert_close(got, truth, rtol=3e-2, atol=3e-2 * np.abs(truth).max(), what="cfg5 vs dequantised f64")


def test_fp8_linear_256_row_tiles_match_dequantised_f64(hip):
    """256 tiles of 256 x 256 fill one round, so the e4m3 GEMM takes its 256-row tile."""
    print("fp8 linear [4096,512] x [4096,512]^T", flush=True)
    rng = np.random.default_rng(12)
    w = (rng.standard_normal((4096, 512), dtype=np.float32) * 0.02).astype(np.float32)
    xbits = f32_to_bf16_bits(rng.standard_normal((4096, 512), dtype=np.float32))
    g, x, y = bench.fp8_graph(K, [4096, 512], w.tobytes(), [4096, 512])
    feeds = {x: Tensor(DType.BF16, [4096, 512], xbits.tobytes())}
    plan = hip.plan(g, [y], feeds)
    assert plan.steps()[-1] == "gemm_mfma_e4m3_nt_256x256 b1 m4096 n4096 k512", plan.steps()
    plan.launch()
    got = to_f32(plan.output(0))
    truth = dequant_f64_linear(xbits, w)
    assert_close(got, truth, rtol=3e-2, atol=3e-2 * np.abs(truth).max(), what="fp8 256-row vs dequantised f64")


# ---------------- 64-bit addressing ----------------

def tiled_bf16(n: int, seed: int, std: float) -> np.ndarray:
    """n bf16 values: a random block of prime length 1,000,003 repeated, so that an address
    that wrapped at 2^31 elements or bytes would read different values."""
    blk = f32_to_bf16_bits(np.random.default_rng(seed).standard_normal(1_000_003, dtype=np.float32) * std)
    return np.resize(blk, n)


def test_gemm_64bit_dma_form_matches_f64(hip):
    """A spans 2^31 bytes: the GEMM loads it with the 64-bit-address DMA form."""
    print("gemm a64 [262144,4096]@[4096,256]", flush=True)
    m, k, n = 262144, 4096, 256
    abits = tiled_bf16(m * k, 21, 1.0 / 64).reshape(m, k)
    bbits = tiled_bf16(k * n, 22, 1.0 / 64).reshape(k, n)
    g = K.Graph()
    a = g.input([m, k], DType.BF16)
    b = g.input([k, n], DType.BF16)
    c = g.matmul(a, b)
    plan = hip.plan(g, [c], {a: Tensor(DType.BF16, [m, k], abits.tobytes()),
                             b: Tensor(DType.BF16, [k, n], bbits.tobytes())})
    assert plan.steps() == [f"gemm_mfma_bf16_nn_256x256_a64 b1 m{m} n{n} k{k}"], plan.steps()
    plan.launch()
    got = to_f32(plan.output(0))
    rows = row_sample(m, 256, 512, 4)
    truth = bf16_bits_to_f32(abits[rows]).astype(np.float64) @ bf16_bits_to_f32(bbits).astype(np.float64)
    assert_close(got[rows], truth, rtol=1e-2, atol=1e-2 * np.abs(truth).max(), what="gemm a64 vs f64")


def test_line_kernel_64bit_indexing_bit_exact(hip):
    """Row max and argmax over a bf16 [65600, 32768] input (2^31 + 2^21 elements): the generated
    kernel indexes in 64 bits; both results are bit-exact."""
    print("line kernel idx64 [65600,32768] bf16", flush=True)
    rows, cols = 65600, 32768
    xbits = tiled_bf16(rows * cols, 23, 3.0).reshape(rows, cols)
    g = K.Graph()
    x = g.input([rows, cols], DType.BF16)
    mx = g.reduce_max(x, 1)
    am = g.argmax(x, 1)
    src = g.codegen([mx, am])
    assert "u64" in src
    got_m, got_a = hip.eval_many_with(g, [mx, am], {x: Tensor(DType.BF16, [rows, cols], xbits.tobytes())})
    for r0 in range(0, rows, 8192):
        xf = bf16_bits_to_f32(xbits[r0:r0 + 8192])
        np.testing.assert_array_equal(got_a.numpy()[r0:r0 + 8192], np.argmax(xf, axis=1))
        np.testing.assert_array_equal(bf16_bits_to_f32(got_m.numpy()[r0:r0 + 8192]), xf.max(axis=1))
