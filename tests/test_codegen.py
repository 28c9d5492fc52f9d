"""Fusion planning and code generation on the CPU (no GPU): every hot-path graph lowers to the
expected number of device steps and each generated kernel compiles for gfx950 with hipRTC."""
import numpy as np
import pytest

import kurumi_amd as K
from kurumi_amd import DType, Graph


def steps(src: str):
    return [l.split(": ", 1)[1] for l in src.splitlines() if l.startswith("// step ")]


def cfg1(n=4096):
    g = Graph()
    x = g.input([n, n], DType.F32)
    b = g.input([n], DType.F32)
    y = g.sum(g.mul(g.relu(g.add(g.mul(x, x), g.broadcast_to(b, [n, n]))), g.scalar(x, 0.5)), 1)
    return g, [y]


def cfg2(dt, decomposed, rows=8192, cols=32000):
    g = Graph()
    x = g.input([rows, cols], dt)
    if decomposed:
        m = g.reduce_max(x, 1)
        e = g.exp(g.sub(x, g.expand(g.reshape(m, [rows, 1]), [rows, cols])))
        y = g.div(e, g.expand(g.reshape(g.sum(e, 1), [rows, 1]), [rows, cols]))
    else:
        y = g.softmax(x, 1)
    return g, [y, g.cast(g.argmax(y, 1), DType.I32)]


def test_cfg1_single_line_kernel_compiles():
    g, roots = cfg1()
    st = steps(g.codegen(roots, compile=True))
    assert len(st) == 1 and st[0].startswith("ku_line_4096x4096")


@pytest.mark.parametrize("dt", [DType.F32, DType.BF16])
@pytest.mark.parametrize("decomposed", [True, False])
def test_cfg2_single_kernel_for_softmax_and_argmax(dt, decomposed):
    g, roots = cfg2(dt, decomposed)
    src = g.codegen(roots, compile=True)
    st = steps(src)
    assert len(st) == 1 and st[0].startswith("ku_line_8192x32000")
    # the line stays in registers: caches for the loaded row, one LDS fold per reduction level
    assert "cache" in src


def test_cfg3_gemm_steps():
    g = Graph()
    c = g.matmul(g.input([4096, 4096], DType.BF16), g.input([4096, 11008], DType.BF16))
    assert steps(g.codegen([c])) == ["gemm_mfma_bf16_nn_256x256 b1 m4096 n11008 k4096"]
    g = Graph()
    c = g.dot_general(g.input([8, 2048, 128], DType.BF16), g.input([8, 128, 2048], DType.BF16), [2], [1], [0], [0])
    assert steps(g.codegen([c])) == ["gemm_mfma_bf16_nn_128x128_persistent b8 m2048 n2048 k128"]
    g = Graph()
    c = g.dot_general(g.input([64, 256], DType.BF16), g.input([128, 256], DType.BF16), [1], [1])
    assert steps(g.codegen([c])) == ["gemm_mfma_bf16_nt_192x256 b1 m64 n128 k256"]
    g = Graph()  # transposed lhs is canonicalised by a copy kernel first
    c = g.dot_general(g.input([256, 64], DType.BF16), g.input([256, 128], DType.BF16), [0], [0])
    st = steps(g.codegen([c], compile=True))
    assert len(st) == 2 and st[0].startswith("ku_ew") and st[1].startswith("gemm_mfma_bf16_nn")


def test_gemm_labels_name_the_tile_and_the_64bit_form():
    g = Graph()  # 2^31 bytes of A: the 64-bit-address DMA form
    c = g.matmul(g.input([262144, 4096], DType.BF16), g.input([4096, 256], DType.BF16))
    assert steps(g.codegen([c])) == ["gemm_mfma_bf16_nn_256x256_a64 b1 m262144 n256 k4096"]
    g = Graph()  # 256 tiles of 256 x 256 fill one round: 256-row tiles
    x = g.input([4096, 512], DType.BF16)
    w = g.constant(np.random.default_rng(0).normal(0, 0.02, (4096, 512)).astype(np.float32))
    st = steps(g.codegen([K.amp_fp8(g, g.dot_general(x, g.cast(w, DType.BF16), [1], [1]))], compile=True))
    assert st[-1] == "gemm_mfma_e4m3_nt_256x256 b1 m4096 n4096 k512"


@pytest.mark.parametrize("fused", [True, False])
def test_cfg4_attention_is_one_step(fused):
    g = Graph()
    q, k, v = (g.input([4, 32, 2048, 128], DType.BF16) for _ in range(3))
    o = g.sdpa_fused(q, k, v, True) if fused else g.sdpa_decomposed(q, k, v, True)
    st = steps(g.codegen([o]))
    assert len(st) == 1 and st[0].startswith("attn") and "causal" in st[0]


def test_decomposed_attention_with_non_causal_bias_is_not_matched():
    g = Graph()
    s = 64
    q, k, v = (g.input([1, 2, s, 32], DType.F32) for _ in range(3))
    raw = g.dot_general(q, k, [3], [3], [0, 1], [0, 1])
    sc = g.mul(raw, g.scalar(raw, 0.125))
    bias = np.zeros((s, s), np.float32)
    bias[0, 5] = -1.0  # not a causal mask
    sc = g.add(sc, g.expand(g.reshape(g.constant(bias), [1, 1, s, s]), [1, 2, s, s]))
    o = g.dot_general(g.softmax(sc, 3), v, [3], [2], [0, 1], [0, 1])
    st = steps(g.codegen([o], compile=True))
    assert not any(x.startswith("attn") for x in st) and len(st) == 3


def misplaced_causal_attention(g, s=64, d=32, dt=DType.F32):
    """Scores [1, s, s, d] whose causal-valued constant is reshaped to [1, s, 1, s]: with H == S
    the shapes line up, but the mask runs along (head, key) instead of (query, key)."""
    q, k, v = (g.input([1, s, s, d], dt) for _ in range(3))
    raw = g.dot_general(q, k, [3], [3], [0, 1], [0, 1])
    sc = g.mul(raw, g.scalar(raw, 1.0 / np.sqrt(d)))
    causal = np.triu(np.full((s, s), -np.inf, np.float32), 1)
    bias = g.expand(g.reshape(g.constant(causal), [1, s, 1, s]), [1, s, s, s])
    if dt != DType.F32:
        bias = g.cast(bias, dt)
    sc = g.add(sc, bias)
    return (q, k, v), g.dot_general(g.softmax(sc, 3), v, [3], [2], [0, 1], [0, 1])


@pytest.mark.parametrize("dt", [DType.F32, DType.BF16])
def test_decomposed_attention_with_misplaced_causal_bias_is_not_matched(dt):
    g = Graph()
    _, o = misplaced_causal_attention(g, dt=dt)
    st = steps(g.codegen([o], compile=True))
    assert not any(x.startswith("attn") for x in st), st


def test_decomposed_attention_bias_with_other_expand_target_is_not_matched():
    # bias broadcast to a larger shape than the scores (the add then broadcasts nothing): the
    # expand target must equal the score shape exactly
    g = Graph()
    s = 64
    q, k, v = (g.input([2, 1, s, 32], DType.F32) for _ in range(3))
    raw = g.dot_general(q, k, [3], [3], [0, 1], [0, 1])
    sc = g.mul(raw, g.scalar(raw, 0.125))
    causal = np.triu(np.full((s, s), -np.inf, np.float32), 1)
    sc = g.add(sc, g.expand(g.reshape(g.constant(causal), [1, 1, s, s]), [2, 1, s, s]))
    o = g.dot_general(g.softmax(sc, 3), v, [3], [2], [0, 1], [0, 1])
    st = steps(g.codegen([o]))
    assert len(st) == 1 and st[0].startswith("attn") and "causal" in st[0]


def test_cfg5_fp8_linear_lowering():
    g = Graph()
    x = g.input([2048, 4096], DType.BF16)
    w = g.constant(np.random.default_rng(0).normal(0, 0.02, (256, 4096)).astype(np.float32))
    y = K.amp_fp8(g, g.dot_general(x, g.cast(w, DType.BF16), [1], [1]))
    assert g.dtype(y) == DType.BF16 and g.shape(y) == (2048, 256)
    st = steps(g.codegen([y], compile=True))
    # weights quantised on the host; on device: the activation quantisation (absmax + quantise,
    # one step) and the fp8 GEMM with both scales in its epilogue
    assert st == ["actq_e4m3 BF16 n8388608", "gemm_mfma_e4m3_nt_192x256 b1 m2048 n256 k4096"]


def test_amp_fp8_host_quantization_matches_numpy():
    import kutest

    rng = np.random.default_rng(1)
    wv = rng.normal(0, 0.02, (16, 64)).astype(np.float32)
    g = Graph()
    x = g.input([4, 64], DType.F32)
    y = K.amp_fp8(g, g.dot_general(x, g.constant(wv), [1], [1]))
    lines = g.dump(y).splitlines()
    wq_id = next(int(l.split()[0][1:]) for l in lines if "Const[16, 64]" in l)
    sw_id = next(int(l.split()[0][1:]) for l in lines if "Const[16]" in l)
    wq = kutest.interpret(g, [wq_id])[0].numpy()
    sw = kutest.interpret(g, [sw_id])[0].numpy()
    np.testing.assert_array_equal(sw, (np.abs(wv).max(1) / np.float32(448)).astype(np.float32))
    want = kutest.cast_bits((wv / sw[:, None]).astype(np.float32), DType.F32, DType.F8E4M3)
    np.testing.assert_array_equal(wq, want)


def test_generic_paths_compile():
    g = Graph()
    x = g.input([5, 6, 7], DType.F32)
    i = g.input([5, 6, 7], DType.I16)
    outs = [g.sum(x, 0), g.reduce_max(x, 1), g.argmax(x, 2), g.prod(g.permute(x, [2, 0, 1]), 1),
            g.cast(g.floor(g.mul(x, g.scalar(x, 3.0))), DType.I8), g.shl(i, i), g.idiv(i, i),
            g.bitcast(g.cast(x, DType.BF16), DType.I16), g.pad(x, [(1, 1), (0, 2), (3, 0)]),
            g.flip(g.slice_step(x, [(0, 5, 2), (1, 6, 1), (0, 7, 3)]), [0, 2]),
            g.where(g.lt(x, g.scalar(x, 0.0)), x, g.neg(x)), g.rmsnorm(x, 2, 1e-6), g.iota([3, 4], 0, DType.F16),
            g.rand_uniform([2, 9], 5)]
    src = g.codegen(outs, compile=True)
    assert len(steps(src)) >= 5


def test_unsupported_dtype_is_an_error_not_a_fallback():
    g = Graph()
    z = g.input([4], DType.C64)
    y = g.add(z, z)
    with pytest.raises(K.KuError, match="complex"):
        g.codegen([y])


# ---------------- movement through computed values, nn chains ----------------

def test_rope_is_one_table_kernel_and_one_fused_kernel():
    """rope (attention.rs:9-36): the [S, D/2] angle table is computed once, everything else --
    two half slices, the negation, both pad+add concats and the broadcast tables -- is one pass."""
    g = Graph()
    x = g.input([4, 32, 2048, 128], DType.F32)
    st = steps(g.codegen([g.rope(x)], compile=True))
    assert len(st) == 2, st
    assert st[0].startswith("ku_ew_2048x64_") and st[1].startswith("ku_ew_4x32x2048x128_")


def test_movement_of_computed_values_stays_in_one_kernel():
    g = Graph()
    x = g.input([64, 96], DType.F32)
    y = g.input([96, 64], DType.F32)
    t = g.add(g.transpose(g.neg(x), 0, 1), y)                        # permute of a computed value
    p = g.pad(g.exp(x), [(1, 2), (0, 4)])                            # pad of a computed value
    c = g.add(g.pad(g.neg(x), [(0, 0), (0, 96)]), g.pad(g.exp(x), [(0, 0), (96, 0)]))  # concat
    f = g.flip(g.slice_step(g.mul(x, x), [(0, 64, 2), (3, 96, 1)]), [0, 1])
    for root in (t, p, c, f):
        st = steps(g.codegen([root], compile=True))
        assert len(st) == 1, (root, st)


def test_broadcast_of_costly_values_is_computed_once():
    g = Graph()
    v = g.input([256], DType.F32)
    big = g.add(g.broadcast_to(g.exp(v), [512, 256]), g.input([512, 256], DType.F32))
    assert len(steps(g.codegen([big]))) == 2
    cheap = g.add(g.broadcast_to(g.neg(v), [512, 256]), g.input([512, 256], DType.F32))
    assert len(steps(g.codegen([cheap]))) == 1


@pytest.mark.parametrize("act", ["silu", "gelu", "sigmoid", "tanh"])
@pytest.mark.parametrize("dt", [DType.F32, DType.BF16])
def test_activation_chains_are_one_kernel(act, dt):
    g = Graph()
    a = g.input([2048, 11008], dt)
    b = g.input([2048, 11008], dt)
    y = g.mul(getattr(g, act)(a), b)  # e.g. the SwiGLU gate silu(a) * b
    st = steps(g.codegen([y], compile=True))
    assert len(st) == 1 and st[0].startswith("ku_ew_2048x11008_"), st


@pytest.mark.parametrize("dt", [DType.F32, DType.BF16])
def test_rmsnorm_is_one_line_kernel(dt):
    g = Graph()
    x = g.input([8192, 4096], dt)
    st = steps(g.codegen([g.rmsnorm(x, 1, 1e-6)], compile=True))
    assert len(st) == 1 and st[0].startswith("ku_line_8192x4096_"), st


def test_rope_rejects_bf16_like_the_reference():
    """The rope tables are f32 (attention.rs:14-15), so `mul(x, cos)` needs an f32 x."""
    g = Graph()
    x = g.input([2, 8, 16], DType.BF16)
    with pytest.raises(K.KuError, match="dtype"):
        g.rope(x)


def _steps(g, roots):
    return [l.split(": ", 1)[1] for l in g.codegen(roots).splitlines() if l.startswith("// step ")]


@pytest.mark.parametrize("d,t", [(DType.BF16, DType.F32), (DType.F16, DType.F32), (DType.BF16, DType.F16),
                                 (DType.F32, DType.BF16), (DType.F32, DType.F16)])
def test_cast_of_a_matmul_rides_in_the_gemm_epilogue(d, t):
    g = Graph()
    a = g.input([256, 128], d)
    b = g.input([128, 512], d)
    y = g.matmul(a, b)
    c = g.cast(y, t)
    steps = _steps(g, [c])
    assert len(steps) == 1 and steps[0].endswith("+cast " + t.name), steps
    # the dot itself requested too: the GEMM writes the dot's dtype and a cast kernel follows
    steps = _steps(g, [y, c])
    assert len(steps) == 2 and "+cast" not in steps[0], steps


def test_widening_cast_feeding_more_work_stays_in_the_region():
    """cast(f16 dot, f32) -> relu: the elementwise kernel reads the 2-byte dot output and does the
    cast itself (fusing would write 4 bytes and read them back)."""
    g = Graph()
    a = g.input([256, 128], DType.F16)
    b = g.input([128, 512], DType.F16)
    r = g.relu(g.cast(g.matmul(a, b), DType.F32))
    steps = _steps(g, [r])
    assert len(steps) == 2 and "+cast" not in steps[0], steps
    # a narrowing cast feeding more work still rides in the GEMM
    g2 = Graph()
    a2 = g2.input([256, 128], DType.F32)
    b2 = g2.input([128, 512], DType.F32)
    r2 = g2.relu(g2.cast(g2.matmul(a2, b2), DType.BF16))
    steps = _steps(g2, [r2])
    assert len(steps) == 2 and steps[0].endswith("+cast BF16"), steps


@pytest.mark.parametrize("rows,cols,dt", [(4096, 4096, DType.F32), (8192, 4096, DType.F32), (64, 32000, DType.F32),
                                          (8192, 32000, DType.BF16), (300, 1000, DType.F32)])
def test_multi_wave_lines_are_one_group_each(rows, cols, dt):
    """A line spread over several waves folds across them through LDS with a barrier: the group
    must hold exactly that line (a second line in the group would read the first line's partials)."""
    import re
    g = Graph()
    x = g.input([rows, cols], dt)
    y = g.sum(g.mul(x, x), 1)
    src = g.codegen([y])
    lb = int(re.search(r"__launch_bounds__\((\d+)\)", src).group(1))
    m = re.search(r"const u32 lane = threadIdx.x % (\d+)u;", src)
    tpl = int(m.group(1))
    if tpl > 64:
        assert lb == tpl, (lb, tpl)
    else:
        assert lb % tpl == 0


def _scaled_fp8_dot(m, n, k, per_row: bool):
    """cast(dot(f32(xq), f32(wq)) * bcast(sx) * bcast(s), bf16) with s a per-column [n] scale
    (reshape [1, n]) or a per-row [m] scale (reshape [m, 1])."""
    g = Graph()
    xq = g.input([m, k], DType.F8E4M3)
    wq = g.input([n, k], DType.F8E4M3)
    sx = g.input([1], DType.F32)
    s = g.input([m] if per_row else [n], DType.F32)
    d = g.dot_general(g.cast(xq, DType.F32), g.cast(wq, DType.F32), [1], [1])
    y1 = g.mul(d, g.expand(g.reshape(sx, [1, 1]), [m, n]))
    y2 = g.mul(y1, g.expand(g.reshape(s, [m, 1] if per_row else [1, n]), [m, n]))
    return g, (xq, wq, sx, s), g.cast(y2, DType.BF16)


def test_fp8_epilogue_matcher_takes_column_scales_only():
    # per-column scale: one fp8 GEMM with the scales in its epilogue
    g, _, y = _scaled_fp8_dot(256, 256, 128, per_row=False)
    st = steps(g.codegen([y], compile=True))
    assert len(st) == 1 and st[0].startswith("gemm_mfma_e4m3_nt"), st
    # a per-row scale on a square output has the same source shape but runs along the other
    # axis: the matcher must decline it (no fp8 GEMM step)
    g, _, y = _scaled_fp8_dot(256, 256, 128, per_row=True)
    st = steps(g.codegen([y], compile=True))
    assert not any(s.startswith("gemm_mfma_e4m3") for s in st), st
