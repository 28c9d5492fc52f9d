"""Device parity of the nn primitives around the configs and of movement through computed values.

rope (kurumi_core/src/graph/ops/nn/attention.rs:9-36), sigmoid / silu / gelu / tanh
(graph/ops/nn/activation.rs:8-44, ops/core/trig.rs:50-58) and rmsnorm (graph/ops/nn/norm.rs:32-39,
interp/nn.rs:73-120) against the oracle; f32 <= 1e-5 relative, bf16 <= 1e-2 (normwise, with an
elementwise bound whose absolute floor is the same fraction of the largest value). Pure data
movement (pads, slices, flips, permutes and their compositions) is bit-exact.
"""
import numpy as np
import pytest

from kurumi_amd import DType, Graph, Tensor
from kutest import assert_close, f32_to_bf16_bits, interpret, randn, rel_err, to_f32

pytestmark = pytest.mark.gpu


def bf16_tensor(x: np.ndarray) -> Tensor:
    return Tensor(DType.BF16, x.shape, f32_to_bf16_bits(x).tobytes())


def close(got: np.ndarray, want: np.ndarray, tol: float, what: str):
    assert rel_err(got, want) <= tol, f"{what}: normwise {rel_err(got, want):.3g}"
    assert_close(got, want, rtol=tol, atol=tol * max(float(np.abs(want).max()), 1e-30), what=what)


# ---------------- rope ----------------

@pytest.mark.parametrize("shape", [(1, 2, 16, 8), (2, 4, 256, 128), (3, 100, 64), (4, 32, 2048, 128)])
def test_rope_matches_oracle_and_closed_form(hip, shape):
    print(f"rope {shape}", flush=True)
    g = Graph()
    x = g.input(list(shape), DType.F32)
    y = g.rope(x)
    xv = randn(list(shape), 91)
    feeds = {x: Tensor.from_numpy(xv)}
    got = hip.eval_with(g, y, feeds).numpy()
    if np.prod(shape) <= 1 << 20:
        want = interpret(g, [y], feeds)[0].numpy()
        close(got, want, 1e-5, "rope vs oracle")
    # closed form in f64: angle[s, i] = s * 10000^(-2i/D), rotate-half pairing (i, i + D/2)
    s_len, d = shape[-2], shape[-1]
    h = d // 2
    ang = np.arange(s_len)[:, None] * (10000.0 ** (-2.0 * np.arange(h) / d))[None, :]
    c, sn = np.cos(ang), np.sin(ang)
    x1, x2 = xv[..., :h].astype(np.float64), xv[..., h:].astype(np.float64)
    truth = np.concatenate([x1 * c - x2 * sn, x2 * c + x1 * sn], axis=-1)
    # the f32 angle s * exp2(i * c * log2 e) carries about six roundings (< 8 * 2^-24 relative,
    # |angle| < S), and cos is sin(angle + pi/2) with one more rounding of the sum: each output
    # is off by at most (|x1| + |x2|) times that angle error
    dang = 8 * s_len * 2.0 ** -24 + s_len * 2.0 ** -24 + 2.0 ** -22
    bound = np.concatenate([np.abs(x1) + np.abs(x2)] * 2, axis=-1) * dang + 1e-7
    err = np.abs(got.astype(np.float64) - truth)
    assert np.all(err <= bound), f"rope vs f64: worst excess {np.max(err - bound):.3g}"
    # position 0 is the identity, and each rotated pair keeps its norm
    np.testing.assert_array_equal(got[..., 0, :], xv[..., 0, :])
    n_in = x1 ** 2 + x2 ** 2
    n_out = got[..., :h].astype(np.float64) ** 2 + got[..., h:].astype(np.float64) ** 2
    assert np.max(np.abs(n_out - n_in) / np.maximum(n_in, 1e-6)) < 1e-4


# ---------------- activations ----------------

@pytest.mark.parametrize("act", ["sigmoid", "silu", "gelu", "tanh"])
@pytest.mark.parametrize("dt", [DType.F32, DType.BF16])
def test_activations_match_oracle(hip, act, dt):
    print(f"{act} {dt.name}", flush=True)
    g = Graph()
    a = g.input([300, 1000], dt)
    b = g.input([300, 1000], dt)
    y = getattr(g, act)(a)
    gate = g.mul(y, b)
    av = randn([300, 1000], 92, std=4.0)
    bv = randn([300, 1000], 93)
    mk = Tensor.from_numpy if dt == DType.F32 else bf16_tensor
    feeds = {a: mk(av), b: mk(bv)}
    got = hip.eval_many_with(g, [y, gate], feeds)
    want = interpret(g, [y, gate], feeds)
    tol = 1e-5 if dt == DType.F32 else 1e-2
    for i, what in enumerate([act, act + " * b"]):
        close(to_f32(got[i]), to_f32(want[i]), tol, what)
    if dt == DType.F32:  # against the textbook functions in f64
        x = av.astype(np.float64)
        ref = {"sigmoid": 1 / (1 + np.exp(-x)), "silu": x / (1 + np.exp(-x)), "tanh": np.tanh(x),
               "gelu": 0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x ** 3)))}[act]
        close(got[0].numpy(), ref, 1e-5, act + " vs f64")


# ---------------- rmsnorm ----------------

@pytest.mark.parametrize("dt", [DType.F32, DType.BF16])
@pytest.mark.parametrize("rows,cols", [(8192, 4096), (7, 1000), (1, 3)])
def test_rmsnorm_matches_oracle(hip, dt, rows, cols):
    print(f"rmsnorm {dt.name} {rows}x{cols}", flush=True)
    g = Graph()
    x = g.input([rows, cols], dt)
    y = g.rmsnorm(x, 1, 1e-6)
    xv = randn([rows, cols], 94, std=3.0)
    feeds = {x: (Tensor.from_numpy(xv) if dt == DType.F32 else bf16_tensor(xv))}
    got = to_f32(hip.eval_with(g, y, feeds))
    xs = to_f32(feeds[x]).astype(np.float64)
    truth = xs / np.sqrt((xs ** 2).mean(axis=1, keepdims=True) + 1e-6)
    tol = 1e-5 if dt == DType.F32 else 1e-2
    close(got, truth, tol, "rmsnorm vs f64")
    if rows * cols <= 1 << 20:
        close(got, to_f32(interpret(g, [y], feeds)[0]), tol, "rmsnorm vs oracle")
    # each row has unit mean square
    ms = (got.astype(np.float64) ** 2).mean(axis=1)
    assert np.all(np.abs(ms - 1) < (1e-4 if dt == DType.F32 else 3e-2))


# ---------------- movement through computed values ----------------

def test_composed_pads_slices_flips_are_bit_exact(hip):
    g = Graph()
    x = g.input([5, 7, 6], DType.F32)
    p = g.pad(x, [(1, 2), (0, 3), (2, 0)])
    outs = [
        g.slice_step(p, [(0, 8, 3), (2, 10, 2), (1, 8, 1)]),          # slice of a pad
        g.pad(g.slice_step(x, [(1, 5, 2), (0, 7, 3), (2, 6, 1)]), [(2, 1), (0, 0), (1, 1)]),  # pad of a slice
        g.flip(p, [0, 2]),                                             # flip of a pad
        g.permute(p, [2, 0, 1]),                                       # permute of a pad
        g.pad(p, [(1, 1), (2, 0), (0, 2)]),                            # pad of a pad
        g.expand(g.reshape(g.pad(g.slice_step(x, [(0, 1, 1), (0, 7, 1), (0, 6, 1)]), [(0, 0), (1, 1), (0, 2)]),
                           [1, 9, 8]), [4, 9, 8]),                     # unit reshape + expand of a pad
        g.reshape(p, [8, 10, 8]),                                      # a padded reshape that needs a copy
        g.pad(g.neg(x), [(1, 0), (0, 2), (3, 1)]),                     # pad of a computed value
        g.add(g.pad(g.neg(x), [(0, 0), (0, 0), (0, 6)]), g.pad(g.mul(x, x), [(0, 0), (0, 0), (6, 0)])),  # concat
        g.flip(g.slice_step(g.transpose(g.neg(x), 0, 2), [(1, 6, 2), (0, 7, 1), (0, 4, 1)]), [0, 1]),  # chain
    ]
    xv = randn([5, 7, 6], 95)
    feeds = {x: Tensor.from_numpy(xv)}
    got = hip.eval_many_with(g, outs, feeds)
    want = interpret(g, outs, feeds)
    for i, (a, b) in enumerate(zip(got, want)):
        np.testing.assert_array_equal(a.numpy(), b.numpy(), err_msg=f"case {i}")


def test_dot_general_of_a_padded_operand(hip):
    """A zero-padded view reaches the GEMM as a materialised operand, not as raw strides."""
    g = Graph()
    a = g.input([30, 40], DType.F32)
    b = g.input([44, 20], DType.F32)
    y = g.matmul(g.pad(a, [(1, 1), (2, 2)]), b)
    av, bv = randn([30, 40], 96), randn([44, 20], 97)
    feeds = {a: Tensor.from_numpy(av), b: Tensor.from_numpy(bv)}
    got = hip.eval_with(g, y, feeds).numpy()
    truth = np.pad(av.astype(np.float64), [(1, 1), (2, 2)]) @ bv.astype(np.float64)
    close(got, truth, 1e-5, "pad @ b")


def test_broadcast_costly_value_computed_once_matches(hip):
    g = Graph()
    v = g.input([256], DType.F32)
    w = g.input([512, 256], DType.F32)
    y = g.add(g.broadcast_to(g.exp(v), [512, 256]), w)
    vv, wv = randn([256], 98), randn([512, 256], 99)
    feeds = {v: Tensor.from_numpy(vv), w: Tensor.from_numpy(wv)}
    close(hip.eval_with(g, y, feeds).numpy(), interpret(g, [y], feeds)[0].numpy(), 1e-6, "bcast exp")
