"""Casts fused into the GEMM epilogue (cast(dot(a, b)) -> one GEMM that rounds to the dot's dtype
and stores the cast's dtype).

The fused result must be bit-identical to the same GEMM followed by a separate cast kernel (the
plan keeps them apart when the dot itself is also requested), and within the dtype bar of the
oracle: bf16/f16 <= 1e-2, f32 products <= 1e-5 before the narrowing cast.
"""
import numpy as np
import pytest

from kurumi_amd import DType, Graph, Tensor
from kutest import assert_close, f32_to_bf16_bits, interpret, randn, to_f32

pytestmark = pytest.mark.gpu


def tensor(x: np.ndarray, dt: DType) -> Tensor:
    if dt == DType.F32:
        return Tensor.from_numpy(x.astype(np.float32))
    if dt == DType.F16:
        return Tensor(DType.F16, x.shape, x.astype(np.float16).tobytes())
    return Tensor(DType.BF16, x.shape, f32_to_bf16_bits(x).tobytes())


PAIRS = [(DType.BF16, DType.F32), (DType.F16, DType.F32), (DType.BF16, DType.F16), (DType.F16, DType.BF16),
         (DType.F32, DType.BF16), (DType.F32, DType.F16)]


@pytest.mark.parametrize("d,t", PAIRS)
@pytest.mark.parametrize("nt", [False, True])
@pytest.mark.parametrize("b,m,k,n", [(1, 256, 128, 512), (1, 37, 64, 29), (3, 128, 64, 96)])
def test_fused_cast_equals_gemm_then_cast(hip, d, t, nt, b, m, k, n):
    print(f"cast epilogue {d.name}->{t.name} nt={nt} {b}x{m}x{k}x{n}", flush=True)
    g = Graph()
    a_shape = [b, m, k] if b > 1 else [m, k]
    b_shape = ([b, n, k] if nt else [b, k, n]) if b > 1 else ([n, k] if nt else [k, n])
    x = g.input(a_shape, d)
    w = g.input(b_shape, d)
    lc, rc = ([2], [2] if nt else [1]) if b > 1 else ([1], [1] if nt else [0])
    bt = ([0], [0]) if b > 1 else ([], [])
    y = g.dot_general(x, w, lc, rc, *bt)
    c = g.cast(y, t)
    feeds = {x: tensor(randn(a_shape, 41, 1.0 / 8), d), w: tensor(randn(b_shape, 42, 1.0 / 8), d)}
    steps = [l for l in g.codegen([c]).splitlines() if l.startswith("// step ")]
    assert len(steps) == 1 and "+cast" in steps[0], steps
    fused = hip.eval_with(g, c, feeds)
    split = hip.eval_many_with(g, [y, c], feeds)[1]  # the dot is a result too: GEMM, then a cast kernel
    assert fused.dtype == t and fused.shape == split.shape
    np.testing.assert_array_equal(np.frombuffer(fused.data, np.uint8), np.frombuffer(split.data, np.uint8))
    want = to_f32(interpret(g, [c], feeds)[0])
    tol = 1e-2
    assert_close(to_f32(fused), want, rtol=tol, atol=tol * np.abs(want).max(), what="fused cast vs oracle")


def test_matmul_in_f16_policy_graph(hip):
    """The graph the reference's amp pass builds (graph/pass/amp.rs:16-40): inputs cast to f16,
    the f16 GEMM, the result cast back to f32 as the output: the back-cast rides in the GEMM."""
    g = Graph()
    a = g.input([192, 256], DType.F32)
    w = g.input([256, 320], DType.F32)
    out = g.cast(g.matmul(g.cast(a, DType.F16), g.cast(w, DType.F16)), DType.F32)
    feeds = {a: Tensor.from_numpy(randn([192, 256], 43, 0.2)), w: Tensor.from_numpy(randn([256, 320], 44, 0.2))}
    steps = [l for l in g.codegen([out]).splitlines() if l.startswith("// step ")]
    assert any("gemm_mfma_f16" in s and "+cast F32" in s for s in steps), steps
    got = hip.eval_with(g, out, feeds).numpy()
    want = interpret(g, [out], feeds)[0].numpy()
    assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what="amp f16 matmul")
    truth = feeds[a].numpy().astype(np.float64) @ feeds[w].numpy().astype(np.float64)
    assert np.abs(got - truth).max() <= 2e-2 * np.abs(truth).max()
