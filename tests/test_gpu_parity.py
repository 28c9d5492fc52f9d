"""Device-vs-oracle parity of the five hot-path configs and the primitives under them.

Bars (the hot path's stated tolerances): integer, bool and index outputs bit-exact; f32 <= 1e-5 relative;
bf16/f16 <= 1e-2 relative; fp8 GEMM <= 3e-2 relative against the dequantised-f64 product.
Floating tolerances are normwise (max|err| / max|ref|) plus an elementwise bound with an
absolute floor of the same relative size, so cancellation near zero does not hide as noise.
Mirrors the reference's `*_matches_cpu` device tests (kurumi_metal/src/tests/*.rs).
"""
import numpy as np
import pytest

from kurumi_amd import DType, Graph, KuError, Tensor
from kutest import (assert_close, bf16_bits_to_f32, bf16_ulp, cast_bits, f32_to_bf16_bits, interpret, rand_range, randn,
                    rel_err, to_f32)

pytestmark = pytest.mark.gpu


def bf16_tensor(x: np.ndarray) -> Tensor:
    return Tensor(DType.BF16, x.shape, f32_to_bf16_bits(x).tobytes())


def f16_tensor(x: np.ndarray) -> Tensor:
    return Tensor(DType.F16, x.shape, x.astype(np.float16).tobytes())


# ---------------- config 1: fused elementwise + reduce ----------------

def cfg1_graph(n: int, m: int):
    g = Graph()
    x = g.input([n, m], DType.F32)
    b = g.input([m], DType.F32)
    xx = g.mul(x, x)
    s = g.add(xx, g.broadcast_to(b, [n, m]))
    r = g.relu(s)
    h = g.mul(r, g.scalar(r, 0.5))
    return g, x, b, g.sum(h, 1)


@pytest.mark.parametrize("n,m", [(64, 4096), (4096, 4096), (3, 100), (1, 7), (3, 300000)])
def test_cfg1_fused_reduce_matches_oracle(hip, n, m):
    print(f"cfg1 n={n} m={m}", flush=True)
    g, x, b, y = cfg1_graph(n, m)
    xv = rand_range([n, m], 11, -1.0, 1.0)
    bv = rand_range([m], 12, -1.0, 1.0)
    feeds = {x: Tensor.from_numpy(xv), b: Tensor.from_numpy(bv)}
    got = hip.eval_with(g, y, feeds).numpy()
    want = interpret(g, [y], feeds)[0].numpy()
    # f64 truth of the same f32 elementwise values
    h = np.maximum(xv * xv + bv[None, :], np.float32(0)) * np.float32(0.5)
    truth = h.astype(np.float64).sum(axis=1)
    assert rel_err(got, truth) <= 1e-5
    assert_close(got, truth, rtol=1e-5, atol=1e-5 * np.abs(truth).max(), what="cfg1 vs f64")
    # the oracle's sequential f32 fold of m terms: up to (m - 1) * 2^-24 relative (first order)
    bar = max(2e-5, 0.05 * m * 2.0**-24)
    assert_close(got, want, rtol=bar, atol=bar * np.abs(want).max(), what="cfg1 vs oracle")


def test_cfg1_is_one_kernel(hip):
    g, x, b, y = cfg1_graph(128, 256)
    feeds = {x: Tensor.from_numpy(np.ones((128, 256), np.float32)), b: Tensor.from_numpy(np.ones(256, np.float32))}
    plan = hip.plan(g, [y], feeds)
    assert len(plan.steps()) == 1, plan.steps()
    plan.launch()
    np.testing.assert_array_equal(plan.output(0).numpy(), np.full(128, 256.0, np.float32))


# ---------------- config 2: softmax + argmax ----------------

def softmax_graph(rows: int, cols: int, dt: DType, decomposed: bool):
    g = Graph()
    x = g.input([rows, cols], dt)
    if decomposed:
        m = g.reduce_max(x, 1)
        mb = g.expand(g.reshape(m, [rows, 1]), [rows, cols])
        e = g.exp(g.sub(x, mb))
        s = g.sum(e, 1)
        y = g.div(e, g.expand(g.reshape(s, [rows, 1]), [rows, cols]))
    else:
        y = g.softmax(x, 1)
    a = g.cast(g.argmax(y, 1), DType.I32)
    return g, x, y, a


@pytest.mark.parametrize("dt", [DType.F32, DType.BF16])
@pytest.mark.parametrize("decomposed", [False, True])
@pytest.mark.parametrize("rows,cols", [(64, 32000), (33, 1000), (5, 7), (6, 200000)])
def test_cfg2_softmax_argmax_matches_oracle(hip, dt, decomposed, rows, cols):
    # (6, 200000): rows longer than the registers hold (800 KB in f32), re-read instead of cached
    print(f"cfg2 {dt.name} decomposed={decomposed} {rows}x{cols}", flush=True)
    g, x, y, a = softmax_graph(rows, cols, dt, decomposed)
    xv = randn([rows, cols], 21, 3.0)
    t = Tensor.from_numpy(xv) if dt == DType.F32 else bf16_tensor(xv)
    feeds = {x: t}
    gy, ga = hip.eval_many_with(g, [y, a], feeds)
    wy, wa = interpret(g, [y, a], feeds)
    # argmax is bit-exact (first index wins ties)
    np.testing.assert_array_equal(ga.numpy(), wa.numpy())
    assert ga.dtype == DType.I32
    if dt == DType.F32:
        # The oracle folds the row sum sequentially in f32 (interp/nn.rs:53-58): for `cols`
        # positive terms that carries up to (cols - 1) * 2^-24 relative error (first order),
        # in practice a few per cent of it (2.9e-4 at 200000 columns). The 1e-5 bar is therefore
        # taken against the f64 softmax of the same inputs, and the oracle difference is bounded
        # at max(1e-4, 0.05 * cols * 2^-24) (1e-4 up to 32000 columns).
        x64 = xv.astype(np.float64)
        e = np.exp(x64 - x64.max(axis=1, keepdims=True))
        truth = e / e.sum(axis=1, keepdims=True)
        assert_close(to_f32(gy), truth, rtol=1e-5, atol=1e-30, what="softmax f32 vs f64")
        oracle_bar = max(1e-4, 0.05 * cols * 2.0**-24)
        assert_close(to_f32(gy), to_f32(wy), rtol=oracle_bar, atol=1e-30, what="softmax f32 vs oracle")
    else:
        # elementwise: 1e-2 of each element plus one bf16 step at its own magnitude (the device
        # rounds at the same primitives as the oracle; only f32 fold orders differ)
        want = to_f32(wy)
        assert_close(to_f32(gy), want, rtol=1e-2, atol=bf16_ulp(want), what="softmax bf16")


def test_cfg2_is_one_kernel(hip):
    for decomposed in (False, True):
        g, x, y, a = softmax_graph(16, 512, DType.BF16, decomposed)
        plan = hip.plan(g, [y, a], {x: bf16_tensor(np.zeros((16, 512), np.float32))})
        assert len(plan.steps()) == 1, plan.steps()


def test_argmax_ties_and_nan_bit_exact(hip):
    # known answer (kurumi_metal/src/tests/device_ops.rs:101-121) plus the tie / NaN rules
    g = Graph()
    x = g.input([6, 4], DType.F32)
    am = g.argmax(x, 1)
    xv = np.array([[3, 1, 4, 1], [5, 9, 2, 6], [1, 1, 1, 1], [np.nan, 5, 7, 1], [2, np.nan, 7, 7],
                   [-np.inf, -np.inf, -np.inf, -np.inf]], np.float32)
    feeds = {x: Tensor.from_numpy(xv)}
    got = hip.eval_with(g, am, feeds).numpy()
    want = interpret(g, [am], feeds)[0].numpy()
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(got[:2], [2, 1])
    np.testing.assert_array_equal(got[2:], [0, 0, 2, 0])


# ---------------- config 3: GEMM ----------------

@pytest.mark.parametrize("m,k,n", [(128, 256, 192), (64, 4096, 11008 // 8), (17, 33, 65)])
def test_cfg3_bf16_gemm_matches_oracle(hip, m, k, n):
    print(f"cfg3 {m}x{k}x{n}", flush=True)
    g = Graph()
    a = g.input([m, k], DType.BF16)
    b = g.input([k, n], DType.BF16)
    c = g.matmul(a, b)
    av = randn([m, k], 31, 1.0 / 64)
    bv = randn([k, n], 32, 1.0 / 64)
    feeds = {a: bf16_tensor(av), b: bf16_tensor(bv)}
    got = to_f32(hip.eval_with(g, c, feeds))
    want = to_f32(interpret(g, [c], feeds)[0])
    truth = bf16_bits_to_f32(f32_to_bf16_bits(av)).astype(np.float64) @ bf16_bits_to_f32(
        f32_to_bf16_bits(bv)).astype(np.float64)
    assert rel_err(got, truth) <= 1e-2
    assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what="gemm vs oracle")


@pytest.mark.parametrize("dt", [DType.BF16, DType.F16])
@pytest.mark.parametrize("nt", [False, True])
@pytest.mark.parametrize("m,k,n", [(300, 192, 520), (256, 128, 256), (1, 64, 8), (513, 320, 264)])
def test_gemm_layouts_and_edges_match_oracle(hip, dt, nt, m, k, n):
    # NN ([k][n] rhs) and NT ([n][k] rhs, the linear-layer layout), tiles cut by M and N
    print(f"gemm {dt.name} nt={nt} {m}x{k}x{n}", flush=True)
    g = Graph()
    a = g.input([m, k], dt)
    b = g.input([n, k] if nt else [k, n], dt)
    c = g.dot_general(a, b, [1], [1] if nt else [0])
    av = randn([m, k], 35, 1.0 / 16)
    bv = randn([n, k] if nt else [k, n], 36, 1.0 / 16)
    mk = f16_tensor if dt == DType.F16 else bf16_tensor
    feeds = {a: mk(av), b: mk(bv)}
    got = to_f32(hip.eval_with(g, c, feeds))
    want = to_f32(interpret(g, [c], feeds)[0])
    assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what="gemm layout")


@pytest.mark.parametrize("dt,nt", [(DType.BF16, False), (DType.F16, True)])
def test_gemm_long_contraction_matches_f64(hip, dt, nt):
    # K = 32768 (512 stages of the MFMA loop) with tiles cut by M and N; the reference is the f64
    # product of the same rounded inputs (the oracle's sequential f32 fold is too slow here)
    m, k, n = 300, 32768, 520
    print(f"gemm long K {dt.name} nt={nt} {m}x{k}x{n}", flush=True)
    g = Graph()
    a = g.input([m, k], dt)
    b = g.input([n, k] if nt else [k, n], dt)
    c = g.dot_general(a, b, [1], [1] if nt else [0])
    mk = f16_tensor if dt == DType.F16 else bf16_tensor
    feeds = {a: mk(randn([m, k], 37, 1.0 / 64)), b: mk(randn([n, k] if nt else [k, n], 38, 1.0 / 4))}
    assert "gemm_mfma" in hip.plan(g, [c], feeds).steps()[0]
    got = to_f32(hip.eval_with(g, c, feeds))
    a64, b64 = to_f32(feeds[a]).astype(np.float64), to_f32(feeds[b]).astype(np.float64)
    want = a64 @ (b64.T if nt else b64)
    assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what="gemm long K")


def test_cfg3_batched_gemm_matches_oracle(hip):
    g = Graph()
    a = g.input([4, 256, 128], DType.BF16)
    b = g.input([4, 128, 192], DType.BF16)
    c = g.dot_general(a, b, [2], [1], [0], [0])
    av = randn([4, 256, 128], 33, 1.0 / np.sqrt(128))
    bv = randn([4, 128, 192], 34, 1.0 / np.sqrt(128))
    feeds = {a: bf16_tensor(av), b: bf16_tensor(bv)}
    got = to_f32(hip.eval_with(g, c, feeds))
    want = to_f32(interpret(g, [c], feeds)[0])
    assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what="batched gemm")


# ---------------- config 4: causal attention ----------------

def attention_graph(shape, dt, causal, fused):
    g = Graph()
    q, k, v = (g.input(list(shape), dt) for _ in range(3))
    o = g.sdpa_fused(q, k, v, causal) if fused else g.sdpa_decomposed(q, k, v, causal)
    return g, q, k, v, o


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("b,h,s,d", [(1, 2, 128, 128), (2, 2, 80, 64), (1, 3, 300, 128), (2, 4, 512, 64),
                                     (1, 1, 64, 32)])
def test_cfg4_attention_matches_oracle(hip, fused, b, h, s, d):
    print(f"cfg4 fused={fused} {b},{h},{s},{d}", flush=True)
    g, q, k, v, o = attention_graph([b, h, s, d], DType.BF16, True, fused)
    feeds = {q: bf16_tensor(randn([b, h, s, d], 41)), k: bf16_tensor(randn([b, h, s, d], 42)),
             v: bf16_tensor(randn([b, h, s, d], 43))}
    got = to_f32(hip.eval_with(g, o, feeds))
    want = to_f32(interpret(g, [o], feeds)[0])
    assert rel_err(got, want) <= 1e-2
    assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what="attention")


@pytest.mark.parametrize("dt,causal,s", [(DType.F16, True, 256), (DType.BF16, False, 200), (DType.F16, False, 64)])
def test_attention_dtypes_and_non_causal_match_oracle(hip, dt, causal, s):
    print(f"attention dt={dt} causal={causal} s={s}", flush=True)
    shape = [1, 2, s, 128]
    g, q, k, v, o = attention_graph(shape, dt, causal, True)
    mk = f16_tensor if dt == DType.F16 else bf16_tensor
    feeds = {q: mk(randn(shape, 51)), k: mk(randn(shape, 52)), v: mk(randn(shape, 53))}
    got = to_f32(hip.eval_with(g, o, feeds))
    want = to_f32(interpret(g, [o], feeds)[0])
    assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what="attention")


@pytest.mark.parametrize("grid", ["8", "16"])
@pytest.mark.parametrize("dt,causal,shape", [(DType.BF16, True, [2, 4, 300, 128]), (DType.BF16, False, [2, 4, 192, 128]),
                                             (DType.F16, True, [1, 8, 520, 64]), (DType.BF16, False, [3, 3, 130, 64]),
                                             (DType.BF16, True, [1, 9, 64, 128])])
def test_attention_persistent_work_groups_match_oracle(hip, monkeypatch, grid, dt, causal, shape):
    # a capped grid gives every work-group several q-tiles in a row (mirrored rounds, tiles of
    # different lengths, odd key-block counts padded to even, partial last tiles), so the
    # pipeline that runs across tile boundaries is checked against the oracle at small shapes
    print(f"attention persistent grid={grid} dt={dt} causal={causal} shape={shape}", flush=True)
    monkeypatch.setenv("KURUMI_HIP_ATTN_GRID", grid)
    g, q, k, v, o = attention_graph(shape, dt, causal, True)
    mk = f16_tensor if dt == DType.F16 else bf16_tensor
    feeds = {q: mk(randn(shape, 61)), k: mk(randn(shape, 62)), v: mk(randn(shape, 63))}
    assert "attn_mfma" in hip.plan(g, [o], feeds).steps()[0]
    got = to_f32(hip.eval_with(g, o, feeds))
    want = to_f32(interpret(g, [o], feeds)[0])
    assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what="attention")


def _attn_grouped_rounds(shape, grid):
    """Rounds of the head-grouped tile order the MFMA kernel takes at this shape and capped grid
    (0 when the shape does not meet its conditions). Mirrors the launcher (grids of whole XCD
    groups) and the kernel's test: grid % (8 * q-tiles) == 0 and heads % (grid / q-tiles) == 0."""
    bh, s = shape[0] * shape[1], shape[2]
    nqt = (s + 127) // 128
    g = min(nqt * bh, grid)
    if g < nqt * bh:
        g = max(8, g & ~7)
    if g % (8 * nqt) or bh % (g // nqt):
        return 0
    return bh // (g // nqt)


@pytest.mark.parametrize("dt,causal,shape,grid", [(DType.BF16, True, [2, 8, 256, 128], 16),
                                                  (DType.F16, True, [2, 8, 256, 64], 16),
                                                  (DType.BF16, True, [1, 16, 384, 64], 24),
                                                  (DType.BF16, False, [1, 24, 200, 128], 16)])
def test_attention_head_grouped_order_matches_oracle(hip, monkeypatch, dt, causal, shape, grid):
    # the tile order cfg 4 runs at full size (every q-tile of a head on one XCD in the same round,
    # odd rounds taking the mirrored q-tile), at small shapes with two and three rounds
    rounds = _attn_grouped_rounds(shape, grid)
    assert rounds >= 2, "shape/grid must take the head-grouped order over several rounds"
    print(f"attention head-grouped grid={grid} rounds={rounds} dt={dt} causal={causal} shape={shape}", flush=True)
    monkeypatch.setenv("KURUMI_HIP_ATTN_GRID", str(grid))
    g, q, k, v, o = attention_graph(shape, dt, causal, True)
    mk = f16_tensor if dt == DType.F16 else bf16_tensor
    feeds = {q: mk(randn(shape, 71)), k: mk(randn(shape, 72)), v: mk(randn(shape, 73))}
    assert "attn_mfma" in hip.plan(g, [o], feeds).steps()[0]
    got = to_f32(hip.eval_with(g, o, feeds))
    want = to_f32(interpret(g, [o], feeds)[0])
    assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what="attention (head-grouped order)")


def test_attention_full_size_mfma_agrees_with_rowwise_kernel(hip, monkeypatch):
    # cfg 4 at its real shape: the MFMA flash kernel against the independent one-query-per-thread
    # kernel (f32 dot products, no MFMA), which the small-shape tests pin to the oracle
    print("cfg4 full size mfma vs rowwise", flush=True)
    shape = [4, 32, 2048, 128]
    g, q, k, v, o = attention_graph(shape, DType.BF16, True, True)
    rng = np.random.default_rng(7)
    feeds = {n: bf16_tensor(rng.standard_normal(shape, dtype=np.float32)) for n in (q, k, v)}
    assert "attn_mfma" in hip.plan(g, [o], feeds).steps()[0]
    fast = to_f32(hip.eval_with(g, o, feeds))
    monkeypatch.setenv("KURUMI_HIP_NO_MFMA", "1")
    g2, q2, k2, v2, o2 = attention_graph(shape, DType.BF16, True, True)
    slow = to_f32(hip.eval_with(g2, o2, {q2: feeds[q], k2: feeds[k], v2: feeds[v]}))
    assert np.isfinite(fast).all()
    assert_close(fast, slow, rtol=1e-2, atol=1e-2 * np.abs(slow).max(), what="attention mfma vs rowwise")


@pytest.mark.parametrize("dt,causal,shape", [(DType.BF16, True, [1, 8, 8192, 128]), (DType.F16, False, [1, 4, 6000, 64])])
def test_attention_long_sequence_mfma_agrees_with_rowwise_kernel(hip, monkeypatch, dt, causal, shape):
    # long rows: a q-tile walks up to 64 key blocks (lazy rescale over many blocks, the pipeline
    # across long tiles), checked against the one-query-per-thread kernel (f32, no MFMA)
    print(f"attention long sequence dt={dt} causal={causal} shape={shape}", flush=True)
    g, q, k, v, o = attention_graph(shape, dt, causal, True)
    rng = np.random.default_rng(11)
    mk = f16_tensor if dt == DType.F16 else bf16_tensor
    feeds = {n: mk(rng.standard_normal(shape, dtype=np.float32)) for n in (q, k, v)}
    assert "attn_mfma" in hip.plan(g, [o], feeds).steps()[0]
    fast = to_f32(hip.eval_with(g, o, feeds))
    monkeypatch.setenv("KURUMI_HIP_NO_MFMA", "1")
    g2, q2, k2, v2, o2 = attention_graph(shape, dt, causal, True)
    slow = to_f32(hip.eval_with(g2, o2, {q2: feeds[q], k2: feeds[k], v2: feeds[v]}))
    assert np.isfinite(fast).all()
    assert_close(fast, slow, rtol=1e-2, atol=1e-2 * np.abs(slow).max(), what="attention long sequence mfma vs rowwise")


def test_attention_causal_prefix_invariance(hip):
    # causality: changing keys/values after position p leaves outputs of queries <= p bit-identical
    shape, p = [1, 4, 1024, 128], 700
    g, q, k, v, o = attention_graph(shape, DType.BF16, True, True)
    rng = np.random.default_rng(8)
    qv, kv, vv = (rng.standard_normal(shape, dtype=np.float32) for _ in range(3))
    a = to_f32(hip.eval_with(g, o, {q: bf16_tensor(qv), k: bf16_tensor(kv), v: bf16_tensor(vv)}))
    kv2, vv2 = kv.copy(), vv.copy()
    kv2[:, :, p + 1:] = rng.standard_normal(kv2[:, :, p + 1:].shape, dtype=np.float32) * 3
    vv2[:, :, p + 1:] = -vv2[:, :, p + 1:]
    b = to_f32(hip.eval_with(g, o, {q: bf16_tensor(qv), k: bf16_tensor(kv2), v: bf16_tensor(vv2)}))
    np.testing.assert_array_equal(a[:, :, :p + 1], b[:, :, :p + 1])
    assert not np.array_equal(a[:, :, p + 1:], b[:, :, p + 1:])


def test_attention_first_query_sees_first_key(hip):
    # tests/ops.rs:256-271: causal query 0 attends only to key 0 -> out[0] == v[0]
    s, dh = 64, 64
    g = Graph()
    q = g.input([1, s, dh], DType.BF16)
    k = g.input([1, s, dh], DType.BF16)
    v = g.input([1, s, dh], DType.BF16)
    o = g.sdpa_fused(q, k, v, True)
    vv = randn([1, s, dh], 44)
    feeds = {q: bf16_tensor(randn([1, s, dh], 45)), k: bf16_tensor(randn([1, s, dh], 46)), v: bf16_tensor(vv)}
    got = to_f32(hip.eval_with(g, o, feeds))
    np.testing.assert_array_equal(got[0, 0], bf16_bits_to_f32(f32_to_bf16_bits(vv[0, 0])))


@pytest.mark.parametrize("dt", [DType.F32, DType.BF16])
def test_attention_with_misplaced_causal_bias_matches_oracle(hip, dt):
    # the causal-valued constant reshaped to [1, S, 1, S] masks along (head, key); the planner
    # must run the decomposed graph as written, not as a causal flash attention
    from test_codegen import misplaced_causal_attention

    print(f"misplaced causal bias dt={dt}", flush=True)
    g = Graph()
    (q, k, v), o = misplaced_causal_attention(g, dt=dt)
    shape = [1, 64, 64, 32]
    mk = bf16_tensor if dt == DType.BF16 else (lambda a: Tensor.from_numpy(a))
    feeds = {q: mk(randn(shape, 71)), k: mk(randn(shape, 72)), v: mk(randn(shape, 73))}
    assert not any("attn" in s for s in hip.plan(g, [o], feeds).steps())
    got = to_f32(hip.eval_with(g, o, feeds))
    want = to_f32(interpret(g, [o], feeds)[0])
    tol = 1e-2 if dt == DType.BF16 else 1e-4
    assert_close(got, want, rtol=tol, atol=tol * np.abs(want).max(), what="misplaced-bias attention")


# ---------------- config 5: fp8 quantized linear ----------------

def test_cfg5_fp8_linear_matches_dequant_f64(hip):
    from kurumi_amd import amp_fp8

    m, k, n = 128, 512, 320
    g = Graph()
    x = g.input([m, k], DType.BF16)
    wv = randn([n, k], 51, 0.02)
    w = g.constant_bytes(DType.F32, wv.astype(np.float32).tobytes(), [n, k])
    y0 = g.dot_general(x, g.cast(w, DType.BF16), [1], [1])
    y = amp_fp8(g, y0)
    xv = randn([m, k], 52)
    feeds = {x: bf16_tensor(xv)}
    got = to_f32(hip.eval_with(g, y, feeds))
    want = to_f32(interpret(g, [y], feeds)[0])
    assert rel_err(got, want) <= 3e-2
    assert_close(got, want, rtol=3e-2, atol=3e-2 * np.abs(want).max(), what="fp8 vs oracle")
    # and the stated oracle of the config: the dequantised-f64 product
    from test_gpu_bench_configs import dequant_f64_linear

    truth = dequant_f64_linear(f32_to_bf16_bits(xv), wv.astype(np.float32))
    assert_close(got, truth, rtol=3e-2, atol=3e-2 * np.abs(truth).max(), what="fp8 vs dequantised f64")


# ---------------- casts, ints, misc primitives (bit-exact) ----------------

@pytest.mark.parametrize("to", [DType.BF16, DType.F16, DType.F8E4M3, DType.F8E5M2, DType.I32, DType.U8, DType.I64,
                                DType.BOOL, DType.F64])
def test_casts_from_f32_bit_exact(hip, to):
    vals = np.concatenate([randn([4000], 61, 50.0), np.array(
        [0.0, -0.0, 1.0, -1.5, 448.0, 449.0, 464.0, 500.0, 1e-9, -1e-9, 3e38, -3e38, np.inf, -np.inf,
         2.5, 3.5, -2.5, 0.5, 65504.0, 65520.0, 1.00390625, 1.01171875, 2 ** -7, 2 ** -10, 57344.0,
         61440.0, 300.7, -129.5, 255.5, 256.0, 4294967296.0], np.float32)])
    g = Graph()
    x = g.input([vals.size], DType.F32)
    c = g.cast(x, to)
    feeds = {x: Tensor.from_numpy(vals)}
    got = hip.eval_with(g, c, feeds).numpy()
    want = interpret(g, [c], feeds)[0].numpy()
    np.testing.assert_array_equal(got, want)


def test_integer_ops_bit_exact(hip):
    g = Graph()
    a = g.input([1000], DType.I32)
    b = g.input([1000], DType.I32)
    outs = [g.add(a, b), g.mul(a, b), g.max(a, b), g.neg(a), g.idiv(a, b), g.bit_and(a, b), g.bit_xor(a, b),
            g.shl(a, b), g.shr(a, b), g.lt(a, b), g.eq(a, b), g.sum(g.reshape(a, [10, 100]), 1),
            g.argmax(g.reshape(a, [10, 100]), 1), g.reduce_max(g.reshape(a, [100, 10]), 0)]
    rng = np.random.default_rng(7)
    av = rng.integers(-2 ** 31, 2 ** 31, 1000, dtype=np.int64).astype(np.int32)
    bv = rng.integers(-40, 40, 1000, dtype=np.int64).astype(np.int32)
    bv[:5] = [0, -1, 0, 31, 33]
    av[:2] = [-2 ** 31, -2 ** 31]
    feeds = {a: Tensor.from_numpy(av), b: Tensor.from_numpy(bv)}
    got = hip.eval_many_with(g, outs, feeds)
    want = interpret(g, outs, feeds)
    for i, (x, y) in enumerate(zip(got, want)):
        np.testing.assert_array_equal(x.numpy(), y.numpy(), err_msg=f"output {i}")


def test_movement_views_match_oracle(hip):
    g = Graph()
    x = g.input([4, 6, 5], DType.F32)
    p = g.permute(x, [2, 0, 1])
    s = g.slice_step(p, [(1, 5, 2), (0, 4, 1), (1, 6, 2)])
    f = g.flip(s, [1])
    pd = g.pad(f, [(1, 0), (0, 2), (1, 1)])
    y = g.add(g.exp(pd), g.scalar(pd, 1.0))
    r = g.sum(g.permute(x, [1, 0, 2]), 0)
    outs = [p, s, f, pd, y, r]
    xv = randn([4, 6, 5], 71)
    feeds = {x: Tensor.from_numpy(xv)}
    got = hip.eval_many_with(g, outs, feeds)
    want = interpret(g, outs, feeds)
    for i in range(4):
        np.testing.assert_array_equal(got[i].numpy(), want[i].numpy(), err_msg=f"view {i}")
    assert_close(got[4].numpy(), want[4].numpy(), rtol=1e-6, atol=0, what="exp(pad)")
    assert_close(got[5].numpy(), want[5].numpy(), rtol=1e-5, atol=1e-6, what="sum axis 0 of permute")


def test_rand_and_iota_on_device(hip):
    g = Graph()
    u = g.rand_uniform([3, 1000], 1234)
    i = g.iota([4, 5], 1, DType.I32)
    got = hip.eval_many_with(g, [u, i], {})
    want = interpret(g, [u, i])
    np.testing.assert_array_equal(got[0].numpy(), want[0].numpy())
    np.testing.assert_array_equal(got[1].numpy(), want[1].numpy())


def test_rmsnorm_and_column_reductions(hip):
    g = Graph()
    x = g.input([37, 300], DType.F32)
    r = g.rmsnorm(x, 1, 1e-6)
    c = g.sum(x, 0)
    mx = g.reduce_max(x, 0)
    xv = randn([37, 300], 81)
    feeds = {x: Tensor.from_numpy(xv)}
    got = hip.eval_many_with(g, [r, c, mx], feeds)
    want = interpret(g, [r, c, mx], feeds)
    assert_close(got[0].numpy(), want[0].numpy(), rtol=1e-5, atol=1e-6, what="rmsnorm")
    assert_close(got[1].numpy(), want[1].numpy(), rtol=1e-5, atol=1e-5, what="col sum")
    np.testing.assert_array_equal(got[2].numpy(), want[2].numpy())


@pytest.mark.parametrize("dt", [DType.F32, DType.BF16])
def test_eval_many_matches_single_eval(hip, dt):
    # backend.rs contract (kurumi_core/tests/engine.rs:228-243): eval_many shares one pass and
    # equals per-node eval bit for bit, on every output
    g, x, y, a = softmax_graph(16, 1000, dt, True)
    s = g.sum(y, 1)
    xv = randn([16, 1000], 91, 3.0)
    feeds = {x: Tensor.from_numpy(xv) if dt == DType.F32 else bf16_tensor(xv)}
    roots = [y, a, s, x]
    many = hip.eval_many_with(g, roots, feeds)
    for i, r in enumerate(roots):
        one = hip.eval_with(g, r, feeds)
        assert many[i].dtype == one.dtype and many[i].shape == one.shape
        np.testing.assert_array_equal(many[i].numpy(), one.numpy(), err_msg=f"output {i}")


@pytest.mark.parametrize("n", [(96 << 20) // 4 + 12345, (8 << 20) // 4 + 3, (4 << 20) // 4 - 1])
def test_large_feeds_and_downloads_are_bit_exact(hip, n):
    # Feeds and results of 4 MiB and more cross the boundary in 32 MiB chunks through two pinned
    # staging buffers: a ragged last chunk, a single partial chunk, and the pageable path below
    # the staging threshold. Two evals in a row reuse the buffers; each must see its own input.
    print(f"staged copies n={n}", flush=True)
    g = Graph()
    x = g.input([n], DType.F32)
    y = g.add(x, g.scalar(x, 1.0))
    for seed in (1, 2):
        xv = np.random.default_rng(seed * n).standard_normal(n, dtype=np.float32)
        got = hip.eval_many_with(g, [y, x], {x: Tensor.from_numpy(xv)})
        np.testing.assert_array_equal(got[1].numpy().view(np.uint32), xv.view(np.uint32))
        np.testing.assert_array_equal(got[0].numpy(), xv + np.float32(1.0))


def test_missing_feed_is_an_error(hip):
    import kurumi_amd as K

    g = Graph()
    x = g.input([4], DType.F32)
    y = g.add(x, x)
    with pytest.raises(K.KuError, match="missing feed"):
        hip.eval_with(g, y, {})


@pytest.mark.parametrize("to", [DType.BF16, DType.F16, DType.F8E4M3, DType.F8E5M2])
def test_f32_to_half_casts_bit_exact_across_the_bit_space(hip, to):
    # every 257th f32 bit pattern (all exponents, signs, NaN payloads, denormals) plus the
    # rounding ties around each half-precision step
    pats = np.arange(0, 2 ** 32, 257, dtype=np.uint64).astype(np.uint32)
    ties = (np.arange(0, 2 ** 16, dtype=np.uint32) << 16) | np.uint32(0x8000)
    bits = np.concatenate([pats, ties, ties + 1, ties - 1])
    vals = bits.view(np.float32)
    g = Graph()
    x = g.input([vals.size], DType.F32)
    c = g.cast(x, to)
    got = hip.eval_with(g, c, {x: Tensor.from_numpy(vals)}).numpy()
    want = cast_bits(vals, DType.F32, to)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("frm", [DType.BF16, DType.F16, DType.F8E4M3, DType.F8E5M2])
@pytest.mark.parametrize("to", [DType.F32, DType.F64, DType.I32])
def test_half_casts_bit_exact_for_every_pattern(hip, frm, to):
    width = 16 if frm in (DType.BF16, DType.F16) else 8
    bits = np.arange(0, 1 << width, dtype=np.uint32).astype(np.uint16 if width == 16 else np.uint8)
    g = Graph()
    x = g.input([bits.size], frm)
    c = g.cast(x, to)
    got = hip.eval_with(g, c, {x: Tensor(frm, [bits.size], bits.tobytes())}).numpy()
    want = cast_bits(bits, frm, to)
    np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8))


# ---------------- empty shapes ----------------

@pytest.mark.parametrize("dt", [DType.F32, DType.BF16])
def test_reductions_over_an_empty_axis_give_the_identity(hip, dt):
    """interp/reduce.rs:67-83 folds from the identity (sum 0, prod 1, max -inf), so an empty
    axis yields it on every line; an empty result stays empty."""
    print(f"empty reductions {dt.name}", flush=True)
    g = Graph()
    x = g.input([3, 0], dt)
    z = g.input([2, 0, 5], dt)
    e = g.input([0, 8], dt)
    outs = [g.sum(x, 1), g.prod(x, 1), g.reduce_max(x, 1), g.sum(z, 1), g.reduce_max(z, 1), g.sum(e, 1), g.add(x, x)]
    mk = (lambda s: Tensor(dt, s, b"")) if dt != DType.F32 else (lambda s: Tensor.from_numpy(np.zeros(s, np.float32)))
    feeds = {x: mk((3, 0)), z: mk((2, 0, 5)), e: mk((0, 8))}
    got = hip.eval_many_with(g, outs, feeds)
    want = interpret(g, outs, feeds)
    for i, (a, b) in enumerate(zip(got, want)):
        assert a.shape == b.shape and a.dtype == b.dtype, (i, a.shape, b.shape)
        np.testing.assert_array_equal(a.numpy(), b.numpy(), err_msg=f"output {i}")


def test_matmul_with_an_empty_contraction_is_zero(hip):
    g = Graph()
    a = g.input([3, 0], DType.F32)
    b = g.input([0, 5], DType.F32)
    y = g.matmul(a, b)
    got = hip.eval_with(g, y, {a: Tensor.from_numpy(np.zeros((3, 0), np.float32)),
                               b: Tensor.from_numpy(np.zeros((0, 5), np.float32))}).numpy()
    np.testing.assert_array_equal(got, np.zeros((3, 5), np.float32))


def test_argmax_over_an_empty_axis_is_an_error(hip):
    """interp/reduce.rs:46 reads element 0 of the axis first (a panic on an empty one)."""
    g = Graph()
    x = g.input([3, 0], DType.F32)
    with pytest.raises(KuError, match="empty axis"):
        hip.eval_with(g, g.argmax(x, 1), {x: Tensor.from_numpy(np.zeros((3, 0), np.float32))})


@pytest.mark.parametrize("per_row", [False, True])
def test_scaled_fp8_dot_square_output_matches_oracle(hip, per_row):
    """A square [m, m] output scaled per row must not be taken for the per-column fp8 epilogue."""
    from test_codegen import _scaled_fp8_dot

    m, k = 256, 128
    g, (xq, wq, sx, s), y = _scaled_fp8_dot(m, m, k, per_row)
    rng = np.random.default_rng(31)
    xb = cast_bits(rng.standard_normal((m, k)).astype(np.float32) * 8, DType.F32, DType.F8E4M3)
    wb = cast_bits(rng.standard_normal((m, k)).astype(np.float32) * 8, DType.F32, DType.F8E4M3)
    feeds = {xq: Tensor(DType.F8E4M3, [m, k], xb.tobytes()), wq: Tensor(DType.F8E4M3, [m, k], wb.tobytes()),
             sx: Tensor.from_numpy(np.array([0.01], np.float32)),
             s: Tensor.from_numpy(np.linspace(0.5, 4.0, m).astype(np.float32))}
    got = to_f32(hip.eval_with(g, y, feeds))
    want = to_f32(interpret(g, [y], feeds)[0])
    assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what=f"scaled fp8 dot per_row={per_row}")


@pytest.mark.parametrize("grid", ["3", "16"])
@pytest.mark.parametrize("dt,nt,b,m,k,n", [(DType.BF16, False, 3, 300, 128, 264), (DType.F16, True, 2, 257, 64, 392),
                                           (DType.BF16, True, 5, 128, 64, 136), (DType.F16, False, 1, 520, 128, 128)])
def test_small_k_gemm_persistent_work_groups_match_oracle(hip, monkeypatch, grid, dt, nt, b, m, k, n):
    # K of one or two 128-byte stages runs on the persistent small-K kernel; a capped grid gives
    # every work-group several tiles in a row (buffer alternation, the waits that let the next
    # tile's loads overtake the previous tile's stores, tiles cut by M and N), checked against
    # the oracle
    print(f"small-K gemm grid={grid} {dt.name} nt={nt} {b}x{m}x{k}x{n}", flush=True)
    monkeypatch.setenv("KURUMI_HIP_SMALLK_GRID", grid)
    g = Graph()
    a = g.input([b, m, k], dt)
    w = g.input([b, n, k] if nt else [b, k, n], dt)
    c = g.dot_general(a, w, [2], [2] if nt else [1], [0], [0])
    mk = f16_tensor if dt == DType.F16 else bf16_tensor
    feeds = {a: mk(randn([b, m, k], 37, 1.0 / 8)), w: mk(randn([b, n, k] if nt else [b, k, n], 38, 1.0 / 8))}
    assert "_persistent" in hip.plan(g, [c], feeds).steps()[0]
    got = to_f32(hip.eval_with(g, c, feeds))
    want = to_f32(interpret(g, [c], feeds)[0])
    assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what="small-K gemm")
