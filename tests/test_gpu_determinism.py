"""Run-to-run determinism: every kernel family returns bit-identical outputs for identical inputs,
on repeated evaluations and on a second backend (fresh plan and constant caches). No kernel on
the path reduces with atomics or in an order that depends on scheduling (persistent work-groups
walk fixed tile sequences; cross-wave and cross-stage sums run in a fixed order), so the check
is exact equality of the raw bytes.
"""
import numpy as np
import pytest

import bench
import kurumi_amd as K
from kurumi_amd import DType, Graph, Tensor
from kutest import f32_to_bf16_bits

pytestmark = pytest.mark.gpu


def _bf16(x: np.ndarray) -> Tensor:
    return Tensor(DType.BF16, x.shape, f32_to_bf16_bits(x.astype(np.float32)).tobytes())


def _cases():
    rng = np.random.default_rng(2024)
    out = []

    g = Graph()
    x, b = g.input([2048, 3000], DType.F32), g.input([3000], DType.F32)
    y = g.sum(g.mul(g.relu(g.add(g.mul(x, x), g.broadcast_to(b, [2048, 3000]))), g.scalar(x, 0.5)), 1)
    out.append(("fused reduce", g, [y], {x: Tensor.from_numpy(rng.uniform(-1, 1, (2048, 3000)).astype(np.float32)),
                                         b: Tensor.from_numpy(rng.uniform(-1, 1, 3000).astype(np.float32))}, None))

    g = Graph()
    x = g.input([512, 32000], DType.F32)
    sm = g.softmax(x, 1)
    out.append(("softmax + argmax", g, [sm, g.cast(g.argmax(sm, 1), DType.I32)],
                {x: Tensor.from_numpy((rng.standard_normal((512, 32000)) * 3).astype(np.float32))}, None))

    g = Graph()
    a, w = g.input([1024, 1024], DType.BF16), g.input([1024, 2560], DType.BF16)
    out.append(("bf16 GEMM (multi-tile)", g, [g.matmul(a, w)],
                {a: _bf16(rng.standard_normal((1024, 1024)) / 32), w: _bf16(rng.standard_normal((1024, 2560)) / 32)},
                None))

    g = Graph()
    a, w = g.input([8, 512, 128], DType.BF16), g.input([8, 128, 512], DType.BF16)
    out.append(("batched small-K GEMM (persistent)", g, [g.dot_general(a, w, [2], [1], [0], [0])],
                {a: _bf16(rng.standard_normal((8, 512, 128)) / 11), w: _bf16(rng.standard_normal((8, 128, 512)) / 11)},
                {"KURUMI_HIP_SMALLK_GRID": "16"}))

    shape = [2, 8, 512, 128]
    g = Graph()
    q, k, v = (g.input(shape, DType.BF16) for _ in range(3))
    out.append(("causal attention (persistent, head-grouped)", g, [g.sdpa_fused(q, k, v, True)],
                {n: _bf16(rng.standard_normal(shape)) for n in (q, k, v)}, {"KURUMI_HIP_ATTN_GRID": "32"}))

    wf = (rng.standard_normal((768, 1024)) * 0.02).astype(np.float32)
    g, x, y = bench.fp8_graph(K, [256, 1024], wf.tobytes(), [768, 1024])
    out.append(("e4m3 linear (absmax, quantise, GEMM)", g, [y], {x: _bf16(rng.standard_normal((256, 1024)))}, None))

    for m, label in ((1, "int4 QuantMatmul GEMV"), (32, "int4 QuantMatmul MFMA")):
        wq = rng.standard_normal((1536, 2048)).astype(np.float32)
        p, s, _ = K.quantize(wq, 4, 128, True)
        g = Graph()
        x = g.input([m, 2048], DType.BF16)
        qw = g.constant_bytes(DType.U8, p.tobytes(), p.shape)
        sc = g.constant_bytes(DType.F16, s.tobytes(), s.shape)
        out.append((label, g, [g.quant_matmul(x, qw, sc, None, 4, 128)],
                    {x: _bf16(rng.standard_normal((m, 2048)))}, None))
    return out


NAMES = ["fused reduce", "softmax + argmax", "bf16 GEMM (multi-tile)", "batched small-K GEMM (persistent)",
         "causal attention (persistent, head-grouped)", "e4m3 linear (absmax, quantise, GEMM)",
         "int4 QuantMatmul GEMV", "int4 QuantMatmul MFMA"]
_BUILT = []


@pytest.mark.parametrize("case", range(len(NAMES)), ids=NAMES)
def test_outputs_are_bit_identical_across_runs_and_backends(hip, monkeypatch, case):
    if not _BUILT:
        _BUILT.extend(_cases())
    assert [c[0] for c in _BUILT] == NAMES
    name, g, roots, feeds, env = _BUILT[case]
    print(f"determinism: {name}", flush=True)
    for key, val in (env or {}).items():
        monkeypatch.setenv(key, val)
    runs = [hip.eval_many_with(g, roots, feeds) for _ in range(3)]
    runs.append(K.HipBackend().eval_many_with(g, roots, feeds))  # fresh caches
    first = [t.numpy().tobytes() for t in runs[0]]
    for i, r in enumerate(runs[1:], 1):
        assert [t.numpy().tobytes() for t in r] == first, f"{name}: run {i} differs from run 0"
