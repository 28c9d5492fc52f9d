"""Builders beyond the five configs' own: the reference's f16 mixed-precision pass (`ku_amp`) and
the decomposed unary / reduction builders (sign, ceil, round, reduce_min, logsumexp,
log_softmax). CPU tests pin the oracle's evaluation of each decomposition against numpy / scipy
and the reference's own amp test; the GPU tests run the device against the oracle."""
import numpy as np
import pytest
from scipy.special import log_softmax as sp_log_softmax, logsumexp as sp_logsumexp

import kurumi_amd as K
from kurumi_amd import DType, Graph, Tensor
from kutest import assert_close, interpret, randn, to_f32, f32_to_bf16_bits


def special_values():
    v = np.array([0.0, -0.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 0.49999997, -0.49999997, 1e-8, -1e-8, 3.7, -3.7,
                  123456.5, -7.0, 8388607.5, 1e30, -1e30, np.inf, -np.inf], np.float32)
    return np.concatenate([v, randn([500], 3, 10.0)])


def test_sign_ceil_round_follow_their_decompositions():
    """elementwise.rs:126-175: sign = select(0<x,1,0) + select(x<0,-1,0); ceil = -floor(-x);
    round = floor(x + 0.5) (half up, not half to even)."""
    x = special_values()
    g = Graph()
    xi = g.input([x.size], DType.F32)
    outs = [g.sign(xi), g.ceil(xi), g.round(xi)]
    got = [t.numpy() for t in interpret(g, outs, {xi: Tensor.from_numpy(x)})]
    np.testing.assert_array_equal(got[0], np.sign(x).astype(np.float32) + np.float32(0))
    np.testing.assert_array_equal(got[1], -np.floor(-x))
    np.testing.assert_array_equal(got[2], np.floor(x + np.float32(0.5)))
    assert got[2][list(x).index(2.5)] == 3.0 and got[2][list(x).index(-2.5)] == -2.0


def test_reduce_min_logsumexp_log_softmax_on_the_oracle():
    x = randn([7, 300], 4, 5.0)
    g = Graph()
    xi = g.input([7, 300], DType.F32)
    outs = [g.reduce_min(xi, 1), g.reduce_min(xi, 0), g.logsumexp(xi, 1), g.log_softmax(xi, 1)]
    got = [t.numpy() for t in interpret(g, outs, {xi: Tensor.from_numpy(x)})]
    np.testing.assert_array_equal(got[0], x.min(axis=1))
    np.testing.assert_array_equal(got[1], x.min(axis=0))
    assert_close(got[2], sp_logsumexp(x.astype(np.float64), axis=1), rtol=1e-5, atol=1e-5, what="logsumexp")
    assert_close(got[3], sp_log_softmax(x.astype(np.float64), axis=1), rtol=1e-5, atol=1e-4, what="log_softmax")


def test_amp_matches_the_reference_test():
    """graph/pass/amp.rs:47-66: the amped graph keeps an f32 output, contracts in f16 and stays
    within 2e-2 of the f32 graph (the reference's constants)."""
    g = Graph()
    a = g.constant((np.sin(np.arange(32) * np.float32(0.1)) * np.float32(0.3)).astype(np.float32).reshape(4, 8))
    b = g.constant((np.cos(np.arange(32) * np.float32(0.2)) * np.float32(0.3)).astype(np.float32).reshape(8, 4))
    c = g.dot_general(a, b, [1], [0])
    y = g.relu(c)
    want = interpret(g, [y])[0].numpy()
    amped = K.amp(g, y)
    assert g.dtype(amped) == DType.F32 and g.dtype(y) == DType.F32
    dump = g.dump(amped)
    assert "Cast { to: F16 }" in dump and "DotGeneral" in dump
    got = interpret(g, [amped])[0].numpy()
    assert np.abs(got - want).max() < 2e-2
    # node order of the rewrite: cast a, cast b, f16 dot, cast back, then the rebuilt relu
    n0 = y + 1
    assert [g.dtype(n0 + i) for i in range(4)] == [DType.F16, DType.F16, DType.F16, DType.F32]
    assert g.shape(n0 + 2) == (4, 4)


def test_amp_leaves_non_f32_contractions_alone():
    g = Graph()
    a = g.input([4, 8], DType.BF16)
    b = g.input([8, 4], DType.BF16)
    c = g.matmul(a, b)
    assert K.amp(g, c) == c


@pytest.mark.parametrize("weight", ["const", "input"])
def test_amp_fp8_all_zero_operands_give_zeros_on_the_oracle(weight):
    """The e4m3 pass divides by 1 where a scale is 0 (an all-zero activation, or an all-zero row
    of an in-graph weight), so the product is 0 there instead of NaN; non-zero inputs are
    quantised exactly as before (the guard passes sx through unchanged)."""
    m, n, k = 4, 6, 128
    rng = np.random.default_rng(2)
    wv = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    wv[2] = 0.0  # an all-zero weight row
    g = Graph()
    x = g.input([m, k], DType.F32)
    if weight == "const":
        w = g.constant(wv)
        feeds_w = {}
    else:
        w = g.input([n, k], DType.F32)
        feeds_w = {w: Tensor.from_numpy(wv)}
    y = K.amp_fp8(g, g.dot_general(x, w, [1], [1]))
    zero = interpret(g, [y], {x: Tensor.from_numpy(np.zeros((m, k), np.float32)), **feeds_w})[0].numpy()
    np.testing.assert_array_equal(zero, np.zeros((m, n), np.float32))
    xv = rng.standard_normal((m, k)).astype(np.float32)
    got = interpret(g, [y], {x: Tensor.from_numpy(xv), **feeds_w})[0].numpy()
    assert np.isfinite(got).all() and (got[:, 2] == 0).all()
    # the unguarded quantisation, restated with numpy: sx = max|x| / 448, xq = e4m3(x * (1/sx))
    import kutest
    sx = np.float32(np.abs(xv).max()) * np.float32(1.0 / 448.0)
    xq = kutest.cast_bits((xv * (np.float32(1.0) / sx)).reshape(-1), DType.F32, DType.F8E4M3)
    xq64 = kutest.cast_bits(xq, DType.F8E4M3, DType.F64).view(np.float64).reshape(m, k)
    assert np.abs(got - (xq64 * np.float64(sx)) @ wv.astype(np.float64).T).max() <= 3e-2 * np.abs(got).max()


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [DType.F32, DType.BF16])
def test_builders_on_device_match_oracle(hip, dt):
    x = special_values()
    x2 = randn([33, 1000], 5, 4.0)
    g = Graph()
    xi = g.input([x.size], dt)
    mi = g.input([33, 1000], dt)
    outs = [g.sign(xi), g.ceil(xi), g.round(xi), g.reduce_min(mi, 1), g.reduce_min(mi, 0), g.logsumexp(mi, 1),
            g.log_softmax(mi, 1)]
    mk = (lambda a: Tensor.from_numpy(a)) if dt == DType.F32 else (
        lambda a: Tensor(DType.BF16, a.shape, f32_to_bf16_bits(a).tobytes()))
    feeds = {xi: mk(x), mi: mk(x2)}
    got = hip.eval_many_with(g, outs, feeds)
    want = interpret(g, outs, feeds)
    for i in range(5):  # exact ops
        np.testing.assert_array_equal(got[i].numpy(), want[i].numpy(), err_msg=f"output {i}")
    tol = 1e-5 if dt == DType.F32 else 1e-2
    for i in (5, 6):
        w = to_f32(want[i])
        assert_close(to_f32(got[i]), w, rtol=tol, atol=tol * np.abs(w).max(), what=f"output {i}")


@pytest.mark.gpu
def test_amp_graph_on_device_matches_oracle(hip):
    """The amped linear runs on the f16 MFMA GEMM; its cast back to f32 joins the relu's region
    (a widening cast that feeds more elementwise work reads the 2-byte GEMM output)."""
    g = Graph()
    x = g.input([96, 256], DType.F32)
    w = g.constant(randn([256, 320], 7, 0.05))
    y = g.relu(g.matmul(x, w))
    amped = K.amp(g, y)
    feeds = {x: Tensor.from_numpy(randn([96, 256], 8))}
    plan = hip.plan(g, [amped], feeds)
    assert any(s.startswith("gemm_mfma_f16") for s in plan.steps()), plan.steps()
    got = hip.eval_with(g, amped, feeds).numpy()
    want = interpret(g, [amped], feeds)[0].numpy()
    assert_close(got, want, rtol=1e-2, atol=1e-2 * np.abs(want).max(), what="amp on device vs oracle")
    f32 = interpret(g, [y], feeds)[0].numpy()
    assert np.abs(got - f32).max() <= 2e-2 * max(1.0, np.abs(f32).max())
