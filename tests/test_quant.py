"""Weight-only quantization: ku_quantize, Op::QuantMatmul's record-time checks, the oracle.

Mirrors kurumi_core/src/quant/tests.rs (round-trip bound in all modes, int8 beats int4, nibble
packing, the op against dequantize-then-matmul) and pins the format itself with exactly
representable weights: the packed bytes (low field first), the f16 scales and the
round-half-away-from-zero rule are checked against values worked out by hand. The dequantizer
used as the independent check here unpacks the bytes with numpy.
"""
import numpy as np
import pytest

import kurumi_amd as K
from kurumi_amd import DType, Graph, KuError, Tensor
from kutest import interpret


def unpack(packed: np.ndarray, cols: int, bits: int) -> np.ndarray:
    """Raw fields [rows, cols] of a packed [rows, cols*bits/8] array (low field first)."""
    per = 8 // bits
    rows = packed.shape[0]
    b = packed.astype(np.uint32).reshape(rows, cols // per, 1)
    shifts = (np.arange(per) * bits).astype(np.uint32).reshape(1, 1, per)
    return ((b >> shifts) & ((1 << bits) - 1)).reshape(rows, cols)


def dequant(packed, scales, mins, cols, bits, group):
    raw = unpack(packed, cols, bits).astype(np.int64)
    s = np.repeat(scales.view(np.float16).astype(np.float32), group, axis=1)
    if mins is None:
        q = np.where(raw >= 1 << (bits - 1), raw - (1 << bits), raw).astype(np.float32)
        return (q * s).astype(np.float32)
    m = np.repeat(mins.view(np.float16).astype(np.float32), group, axis=1)
    return (raw.astype(np.float32) * s).astype(np.float32) + m


def quant_graph(act: np.ndarray, packed, scales, mins, bits, group, act_dtype=DType.F32):
    g = Graph()
    if act_dtype == DType.F32:
        a = g.constant(act.astype(np.float32))
    else:
        a = g.cast(g.constant(act.astype(np.float32)), act_dtype)
    qw = g.constant_bytes(DType.U8, packed.tobytes(), packed.shape)
    sc = g.constant_bytes(DType.F16, scales.tobytes(), scales.shape)
    mn = None if mins is None else g.constant_bytes(DType.F16, mins.tobytes(), mins.shape)
    return g, g.quant_matmul(a, qw, sc, mn, bits, group)


# ---------------- the quantizer (quant.rs:43-91) ----------------

@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("sym", [True, False])
def test_roundtrip_bound_all_modes(bits, group, sym):
    """quant/tests.rs:5-29: every element comes back within half a step (plus f16 slack)."""
    rows, cols = 3, 128
    w = ((np.arange(rows * cols) * 37 % 211) / 211.0 - 0.5).astype(np.float32).reshape(rows, cols) * 6.0
    p, s, m = K.quantize(w, bits, group, sym)
    dq = dequant(p, s, m, cols, bits, group)
    step = np.repeat(s.view(np.float16).astype(np.float32), group, axis=1)
    assert np.all(np.abs(w - dq) <= step * 0.55 + 1e-3)


def test_int8_asym_beats_int4():
    w = (np.sin(np.arange(128, dtype=np.float32)) * 3.0).reshape(2, 64)
    def mse(bits):
        p, s, m = K.quantize(w, bits, 32, False)
        return float(np.mean((w - dequant(p, s, m, 64, bits, 32)) ** 2))
    assert mse(8) < mse(4)


def test_packing_layout_and_scale_exact():
    """Exactly representable int4 weights: amax 3.5 -> scale 3.5/7 = 0.5 (exact in f16), q = 2w,
    fields low nibble first."""
    q = np.array(list(range(-7, 8)) + [0], np.int64)           # 16 values
    w = (0.5 * q).astype(np.float32).reshape(1, 16)
    p, s, m = K.quantize(w, 4, 16, True)
    assert m is None and s.view(np.float16)[0, 0] == np.float16(0.5)
    nib = q & 15
    want = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
    np.testing.assert_array_equal(p[0], want)
    np.testing.assert_array_equal(dequant(p, s, m, 16, 4, 16), w)


def test_asymmetric_layout_exact():
    """w = 1 + q/4 for q = 0..15: min 1.0 and scale (4.75 - 1)/15 = 0.25 are exact, q is recovered."""
    q = np.arange(16)
    w = (1.0 + 0.25 * q).astype(np.float32).reshape(1, 16)
    p, s, m = K.quantize(w, 4, 16, False)
    assert s.view(np.float16)[0, 0] == np.float16(0.25) and m.view(np.float16)[0, 0] == np.float16(1.0)
    np.testing.assert_array_equal(unpack(p, 16, 4)[0], q)
    # int2 fields: four per byte, lowest first
    p2, s2, m2 = K.quantize(np.array([[0, 1, 2, 3, 3, 2, 1, 0]], np.float32), 2, 8, False)
    assert s2.view(np.float16)[0, 0] == np.float16(1.0)
    np.testing.assert_array_equal(p2[0], [0 | 1 << 2 | 2 << 4 | 3 << 6, 3 | 2 << 2 | 1 << 4 | 0 << 6])


def test_rounding_is_half_away_from_zero():
    """int8 symmetric with amax 127 has scale 1.0: x.5 rounds away from zero (f32::round)."""
    w = np.array([[127.0, 2.5, -2.5, 0.5, -0.5, 1.49, -1.51] + [0.0] * 9], np.float32)
    p, s, _ = K.quantize(w, 8, 16, True)
    assert s.view(np.float16)[0, 0] == np.float16(1.0)
    np.testing.assert_array_equal(p[0, :7].view(np.int8), [127, 3, -3, 1, -1, 1, -2])


def test_quantize_rejects_bad_arguments():
    w = np.zeros((2, 64), np.float32)
    with pytest.raises(KuError):
        K.quantize(w, 3, 32, True)
    with pytest.raises(KuError):
        K.quantize(w, 4, 48, True)


# ---------------- Op::QuantMatmul on the oracle ----------------

@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("sym", [True, False])
def test_oracle_matches_dequant_then_matmul(bits, sym):
    """quant/tests.rs:55-74 via the op: equals dequantize-then-matmul (f64 here)."""
    m, n, k, grp = 3, 5, 64, 32
    w = ((np.arange(n * k) * 29 % 83) / 83.0 - 0.5).astype(np.float32).reshape(n, k) * 3.0
    act = ((np.arange(m * k) * 11 % 61) / 61.0 - 0.3).astype(np.float32).reshape(m, k)
    p, s, mn = K.quantize(w, bits, grp, sym)
    g, y = quant_graph(act, p, s, mn, bits, grp)
    got = interpret(g, [y])[0].numpy()
    want = act.astype(np.float64) @ dequant(p, s, mn, k, bits, grp).astype(np.float64).T
    assert np.max(np.abs(got - want)) < 1e-4


def test_quant_matmul_op_matches_reference_case():
    """quant/tests.rs:78-112: int4 asymmetric, the reference's weights and activations."""
    m, n, k, grp = 2, 3, 64, 32
    w = ((np.arange(n * k) * 13 % 97) / 97.0 - 0.5).astype(np.float32).reshape(n, k) * 4.0
    act = ((np.arange(m * k) * 7 % 53) / 53.0).astype(np.float32).reshape(m, k)
    p, s, mn = K.quantize(w, 4, grp, False)
    g, y = quant_graph(act, p, s, mn, 4, grp)
    got = interpret(g, [y])[0].numpy()
    want = act.astype(np.float64) @ dequant(p, s, mn, k, 4, grp).astype(np.float64).T
    assert np.max(np.abs(got - want)) < 1e-3
    full = act.astype(np.float64) @ w.astype(np.float64).T
    assert np.abs(got - full).sum() / max(np.abs(full).sum(), 1e-6) < 0.15


def test_quant_matmul_keeps_act_dtype():
    act = np.ones((2, 32), np.float32)
    p, s, mn = K.quantize(np.ones((4, 32), np.float32), 8, 32, True)
    for dt in (DType.F32, DType.BF16, DType.F16):
        g, y = quant_graph(act, p, s, mn, 8, 32, dt)
        assert g.dtype(y) == dt and g.shape(y) == (2, 4)


def test_quant_matmul_record_time_errors():
    """graph/ops/core/contract.rs:60-110, each check."""
    g = Graph()
    a = g.input([2, 64], DType.F32)
    qw = g.input([4, 32], DType.U8)
    sc = g.input([4, 2], DType.F16)
    ok = g.quant_matmul(a, qw, sc, None, 4, 32)
    assert g.shape(ok) == (2, 4)
    cases = [
        (lambda: g.quant_matmul(a, qw, sc, None, 3, 32), "bits 3"),
        (lambda: g.quant_matmul(a, qw, sc, None, 4, 48), "multiple of group_size"),
        (lambda: g.quant_matmul(a, g.input([4, 16], DType.U8), sc, None, 4, 32), "qweight cols"),
        (lambda: g.quant_matmul(a, g.input([4, 32], DType.I8), sc, None, 4, 32), "qweight must be U8"),
        (lambda: g.quant_matmul(a, qw, g.input([4, 2], DType.F32), None, 4, 32), "scales must be F16"),
        (lambda: g.quant_matmul(g.input([2, 64], DType.I32), qw, sc, None, 4, 32), "act must be float"),
        (lambda: g.quant_matmul(g.input([64], DType.F32), qw, sc, None, 4, 32), "rank-2"),
        (lambda: g.quant_matmul(a, qw, g.input([4, 3], DType.F16), None, 4, 32), "scales must have"),
        (lambda: g.quant_matmul(a, qw, sc, g.input([4, 1], DType.F16), 4, 32), "mins must have"),
    ]
    for f, msg in cases:
        with pytest.raises(KuError, match=msg):
            f()


def test_plan_picks_the_mfma_kernel_for_int4_batches():
    rng = np.random.default_rng(4)
    w = rng.standard_normal((64, 256)).astype(np.float32)
    cases = [(4, 128, DType.BF16, 16, "quant_mfma"), (4, 64, DType.F16, 64, "quant_mfma"),
             (4, 128, DType.BF16, 65, "quant_dequant+gemm"), (4, 128, DType.F32, 16, "quant_dequant+gemm"),
             (8, 128, DType.BF16, 16, "quant_dequant+gemm"), (4, 32, DType.BF16, 16, "quant_dequant+gemm")]
    for bits, group, dt, m, want in cases:
        p, s, mn = K.quantize(w, bits, group, True)
        g, y = quant_graph(rng.standard_normal((m, 256)).astype(np.float32), p, s, mn, bits, group, dt)
        src = g.codegen([y])
        steps = [l.split(": ", 1)[1] for l in src.splitlines() if l.startswith("// step ")]
        assert any(st.startswith(want) for st in steps), (bits, group, dt, m, steps)


def test_plan_labels_gemv_and_gemm_paths():
    rng = np.random.default_rng(3)
    p, s, mn = K.quantize(rng.standard_normal((64, 128)).astype(np.float32), 4, 32, True)
    for m, want in ((1, "quant_gemv int4s g32 m1 n64 k128"), (4, "quant_gemv"), (8, "quant_gemv"), (9, "quant_dequant+gemm"),
                    (65, "quant_dequant+gemm")):
        g, y = quant_graph(rng.standard_normal((m, 128)).astype(np.float32), p, s, mn, 4, 32, DType.BF16)
        src = g.codegen([y])
        steps = [l.split(": ", 1)[1] for l in src.splitlines() if l.startswith("// step ")]
        assert any(st.startswith(want) for st in steps), steps
