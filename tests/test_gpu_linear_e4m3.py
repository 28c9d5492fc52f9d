"""ku_hip_linear_e4m3: the e4m3 linear on caller-owned device buffers.

It runs the same kernels as the graph path (the activation-quantisation step and the fp8 GEMM
the planner lowers ku_amp_fp8's graph to), so its output equals the graph's bit for bit, and
the dequantised-f64 product within the e4m3 bar (3e-2)."""
import numpy as np
import pytest

import bench
import kurumi_amd as K
from hipmem import DevBuf, synchronize
from kurumi_amd import DType, Tensor
from kutest import assert_close, bf16_bits_to_f32, cast_bits, f32_to_bf16_bits
from test_gpu_bench_configs import dequant_f64_linear

pytestmark = pytest.mark.gpu


def quantise_rows(w: np.ndarray):
    """The e4m3 pass's host quantisation of a constant weight: sw = max|w| / 448 per row."""
    sw = (np.abs(w).max(axis=1) / np.float32(448.0)).astype(np.float32)
    sw[~(sw > 0)] = 1.0
    wq = cast_bits(np.ascontiguousarray(w / sw[:, None], dtype=np.float32).reshape(-1), DType.F32,
                   DType.F8E4M3).reshape(w.shape)
    return wq, sw


def run_direct(hip, xbits, x_dtype, wq, sw, y_dtype, m, n, k):
    dx, dwq, dsw = DevBuf.from_numpy(xbits), DevBuf.from_numpy(wq), DevBuf.from_numpy(sw)
    dy = DevBuf(m * n * y_dtype.width)
    hip.linear_e4m3(dx.ptr, x_dtype, dwq.ptr, dsw.ptr, dy.ptr, y_dtype, m, n, k)
    synchronize()
    return dy.numpy(y_dtype.storage, (m, n))


@pytest.mark.parametrize("m,n,k", [(2048, 11008, 4096), (300, 520, 384), (1, 256, 128)])
def test_linear_e4m3_matches_graph_path_bit_for_bit(hip, m, n, k):
    print(f"linear_e4m3 {m}x{n}x{k}", flush=True)
    rng = np.random.default_rng(m + n + k)
    w = (rng.standard_normal((n, k), dtype=np.float32) * 0.02).astype(np.float32)
    xbits = f32_to_bf16_bits(rng.standard_normal((m, k), dtype=np.float32))
    wq, sw = quantise_rows(w)
    got = run_direct(hip, xbits, DType.BF16, wq, sw, DType.BF16, m, n, k)
    g, x, y = bench.fp8_graph(K, [m, k], w.tobytes(), [n, k])
    plan = hip.plan(g, [y], {x: Tensor(DType.BF16, [m, k], xbits.tobytes())})
    assert [s.split(" ")[0] for s in plan.steps()] == ["actq_e4m3", plan.steps()[-1].split(" ")[0]]
    plan.launch()
    np.testing.assert_array_equal(got, plan.output(0).numpy())
    truth = dequant_f64_linear(xbits, w)
    gf = bf16_bits_to_f32(got)
    assert_close(gf, truth, rtol=3e-2, atol=3e-2 * np.abs(truth).max(), what="linear_e4m3 vs dequantised f64")


@pytest.mark.parametrize("x_dtype,y_dtype", [(DType.F16, DType.F32), (DType.F32, DType.F16)])
def test_linear_e4m3_dtypes(hip, x_dtype, y_dtype):
    m, n, k = 96, 320, 256
    rng = np.random.default_rng(5)
    x = rng.standard_normal((m, k), dtype=np.float32) * 3
    xs = x.astype(np.float16) if x_dtype == DType.F16 else x
    w = (rng.standard_normal((n, k), dtype=np.float32) * 0.05).astype(np.float32)
    wq, sw = quantise_rows(w)
    got = run_direct(hip, xs.view(x_dtype.storage), x_dtype, wq, sw, y_dtype, m, n, k)
    gf = got.view(np.float16).astype(np.float32) if y_dtype == DType.F16 else got
    # the dequantised product from the input as given (f16 / f32 values)
    xin = xs.astype(np.float32)
    sx = np.float32(np.abs(xin).max()) * np.float32(1.0 / 448.0)
    xq = cast_bits((xin * (np.float32(1.0) / sx)).reshape(-1), DType.F32, DType.F8E4M3)
    xq64 = cast_bits(xq, DType.F8E4M3, DType.F64).view(np.float64).reshape(m, k)
    wq64 = cast_bits(wq.reshape(-1), DType.F8E4M3, DType.F64).view(np.float64).reshape(n, k)
    truth = (xq64 @ wq64.T) * np.float64(sx) * sw.astype(np.float64)[None, :]
    assert_close(gf, truth, rtol=3e-2, atol=3e-2 * np.abs(truth).max(), what="linear_e4m3 dtypes")


def test_linear_e4m3_all_zero_activation_gives_zeros(hip):
    """sx = max|x| / 448 = 0: both the entry point and the graph path divide by 1 instead, so
    xq = 0 and y = 0 (not 0 * inf = NaN), and they still agree bit for bit."""
    m, n, k = 64, 256, 256
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((n, k), dtype=np.float32) * 0.02).astype(np.float32)
    xbits = np.zeros((m, k), np.uint16)
    wq, sw = quantise_rows(w)
    got = run_direct(hip, xbits, DType.BF16, wq, sw, DType.BF16, m, n, k)
    np.testing.assert_array_equal(got, np.zeros((m, n), np.uint16))
    g, x, y = bench.fp8_graph(K, [m, k], w.tobytes(), [n, k])
    plan = hip.plan(g, [y], {x: Tensor(DType.BF16, [m, k], xbits.tobytes())})
    assert plan.steps()[0].startswith("actq_e4m3"), plan.steps()
    plan.launch()
    np.testing.assert_array_equal(plan.output(0).numpy(), got)
    # and a non-zero x afterwards on the same buffers' path still matches the graph
    xbits = f32_to_bf16_bits(rng.standard_normal((m, k), dtype=np.float32))
    got = run_direct(hip, xbits, DType.BF16, wq, sw, DType.BF16, m, n, k)
    plan.feed(x, Tensor(DType.BF16, [m, k], xbits.tobytes()))
    plan.launch()
    np.testing.assert_array_equal(plan.output(0).numpy(), got)


def test_linear_e4m3_rejects_bad_arguments(hip):
    d = DevBuf(4096)
    with pytest.raises(K.KuError, match="multiple of 128"):
        hip.linear_e4m3(d.ptr, DType.BF16, d.ptr, d.ptr, d.ptr, DType.BF16, 4, 4, 100)
    with pytest.raises(K.KuError, match="null device pointer"):
        hip.linear_e4m3(0, DType.BF16, d.ptr, d.ptr, d.ptr, DType.BF16, 4, 4, 128)
    with pytest.raises(K.KuError, match="x dtype"):
        hip.linear_e4m3(d.ptr, DType.I32, d.ptr, d.ptr, d.ptr, DType.BF16, 4, 4, 128)
