"""Pin the oracle (CPU restatement of kurumi's interpreter) before trusting it.

Each check is chosen so that a plausible restatement mistake fails it: the reference's own
known answers (tests/golden/reference_known_answers.json, each with its file:line), closed
forms, exhaustive round trips, independent implementations (numpy, brute force) and
realize == interpret bit-exactness. CPU only.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from kurumi_amd import DType, Graph, Tensor
from kutest import (assert_close, bf16_bits_to_f32, cast_bits, f32_to_bf16_bits, interpret, oracle, rand_uniform,
                    realize, to_f32)

KA = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


def const(g, a, dt=DType.F32):
    a = np.asarray(a, dtype=np.float32)
    if dt == DType.F32:
        return g.constant(a)
    if dt == DType.BF16:
        return g.constant_bytes(DType.BF16, f32_to_bf16_bits(a).tobytes(), a.shape)
    return g.constant_bytes(dt, cast_bits(a, DType.F32, dt).tobytes(), a.shape)


def run(g, n, feeds=None):
    return interpret(g, [n], feeds)[0]


# ---------------- RNG ----------------

def test_threefry_known_answers():
    for kat in KA["threefry2x32"]:
        assert oracle().kuo_threefry2x32(kat["key"], kat["counter"]) == int(kat["out"], 16), kat["cite"]


def test_uniform_closed_form_and_range():
    u = rand_uniform(42, 10000)
    bits = np.array([oracle().kuo_threefry2x32(42, i) for i in range(100)], dtype=np.uint64)
    expect = ((bits & 0xFFFFFFFF) >> 8).astype(np.float64) / 2 ** 24
    np.testing.assert_array_equal(u[:100].astype(np.float64), expect)
    assert ((u >= 0) & (u < 1)).all() and abs(u.mean() - 0.5) < 0.02
    assert not np.array_equal(u, rand_uniform(43, 10000))


def test_randn_moments():
    from kutest import randn

    x = randn([200000], 9)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01


@pytest.mark.parametrize("seed", [0, 9, 0xFFFF_FFFF_FFFF_FFFF])
def test_randn_is_box_muller_over_the_two_pinned_streams(seed):
    """graph/ops/core/random.rs:28-40: sqrt(-2 ln max(u1, 1e-7)) * cos(2 pi u2), u1 from `seed`
    and u2 from `seed ^ 0xD1B5_4A32_D192_ED03`, each the KAT-pinned uniform map. Recomputed
    here in f64 from those uniforms; the oracle's f32 primitive chain (ln through log2, cos as
    sin(x + pi/2)) stays within a few f32 ulps of it. A wrong stream constant, a swapped branch
    (sin) or a dropped clamp fails."""
    from kutest import rand_uniform, randn

    n = 50000
    x = randn([n], seed).astype(np.float64)
    u1 = rand_uniform(seed, n).astype(np.float64)
    u2 = rand_uniform(seed ^ 0xD1B54A32D192ED03, n).astype(np.float64)
    want = np.sqrt(-2.0 * np.log(np.maximum(u1, np.float64(np.float32(1e-7))))) * np.cos(2.0 * np.pi * u2)
    err = np.abs(x - want)
    assert (err <= 4e-6 * np.maximum(1.0, np.abs(want))).all(), err.max()
    # the clamp binds exactly where the first stream is below 1e-7
    assert np.abs(want).max() < 5.7


# ---------------- conversions ----------------

def test_bf16_round_trip_exhaustive_and_ties():
    bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    f = bf16_bits_to_f32(bits)
    finite = np.isfinite(f)
    back = cast_bits(f[finite], DType.F32, DType.BF16)
    np.testing.assert_array_equal(back, bits[finite])
    # exact midpoints between consecutive bf16 values round to the even mantissa
    lo = bf16_bits_to_f32(np.array([0x3F80, 0x3F81, 0x4000], np.uint16))
    mid = (lo.view(np.uint32) + 0x8000).view(np.float32)
    got = cast_bits(mid, DType.F32, DType.BF16)
    np.testing.assert_array_equal(got, [0x3F80, 0x3F82, 0x4000])
    nan = cast_bits(np.array([np.nan], np.float32), DType.F32, DType.BF16)
    assert (nan[0] & 0x7F80) == 0x7F80 and (nan[0] & 0x7F) != 0


def test_f16_matches_numpy():
    x = np.concatenate([np.random.default_rng(1).normal(0, 300, 100000).astype(np.float32),
                        np.array([65504, 65520, 65519.99, 1e-8, 6.1e-5, -0.0, np.inf], np.float32)])
    got = cast_bits(x, DType.F32, DType.F16).view(np.float16)
    np.testing.assert_array_equal(got, x.astype(np.float16))


def test_nan_payloads_follow_the_half_crate():
    # Casts go through f64 (kurumi_core/src/dtype/convert.rs:14-70) with the half crate's
    # conversions: a NaN keeps its sign and its top mantissa bits and gets the quiet bit. For quiet
    # NaNs that is exactly numpy's rule (npy_floatbits_to_halfbits / npy_halfbits_to_floatbits),
    # so numpy pins the payload shift in both directions; signalling NaNs additionally get the
    # quiet bit (0x200 in f16, 0x400000 in f32), which numpy does not add.
    rng = np.random.default_rng(5)
    man = rng.integers(0, 1 << 22, 4000, dtype=np.uint32)
    sign = rng.integers(0, 2, 4000, dtype=np.uint32) << 31
    qnan = (sign | np.uint32(0x7FC00000) | man).view(np.float32)
    got = cast_bits(qnan, DType.F32, DType.F16)
    np.testing.assert_array_equal(got, qnan.astype(np.float16).view(np.uint16))
    snan = (sign | np.uint32(0x7F800000) | (man | 1)).view(np.float32)  # quiet bit clear
    got = cast_bits(snan, DType.F32, DType.F16)
    want = snan.astype(np.float16).view(np.uint16) | np.uint16(0x0200)
    # numpy turns an all-zero kept payload into 1 to stay a NaN; half's quiet bit already does
    empty = ((snan.view(np.uint32) & np.uint32(0x7FFFFF)) >> 13) == 0
    want = np.where(empty, (sign >> 16).astype(np.uint16) | np.uint16(0x7E00), want)
    np.testing.assert_array_equal(got, want)
    h = (np.uint16(0x7E00) | (rng.integers(0, 1 << 9, 4000, dtype=np.uint16))) | (
        rng.integers(0, 2, 4000, dtype=np.uint16) << 15)
    got = cast_bits(h, DType.F16, DType.F32).view(np.uint32)
    np.testing.assert_array_equal(got, h.view(np.float16).astype(np.float32).view(np.uint32))
    # bf16 <-> f32: the upper half of the f32 pattern, quiet bit (0x40) forced on the way down
    b = cast_bits(snan, DType.F32, DType.BF16)
    np.testing.assert_array_equal(b, (snan.view(np.uint32) >> 16).astype(np.uint16) | np.uint16(0x40))


def _e4m3_table():
    v = np.array([cast_bits(np.array([b], np.uint8), DType.F8E4M3, DType.F64)[0] for b in range(256)])
    return v


def test_e4m3_decode_and_round_trip():
    v = _e4m3_table()
    assert v[0x7E] == 448.0 and v[0x01] == 2.0 ** -9 and v[0x08] == 2.0 ** -6 and np.isnan(v[0x7F])
    codes = np.array([b for b in range(256) if not np.isnan(v[b])], np.uint8)
    back = cast_bits(v[codes].astype(np.float32), DType.F32, DType.F8E4M3)
    want = codes.copy()
    want[want == 0x80] = 0x80  # -0 keeps its sign
    np.testing.assert_array_equal(back, want)
    # representable round trip asserted by the reference
    x = np.array(KA["fp8_round_trip"]["x"], np.float32)
    np.testing.assert_array_equal(cast_bits(cast_bits(x, DType.F32, DType.F8E4M3), DType.F8E4M3, DType.F32), x)


def test_e4m3_brute_force_nearest_even_saturating():
    v = _e4m3_table()
    pos = v[:0x7F]
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.uniform(-500, 500, 20000), rng.uniform(-0.02, 0.02, 20000),
                        (pos[1:] + pos[:-1]) / 2]).astype(np.float32)
    got = cast_bits(x, DType.F32, DType.F8E4M3)
    a = np.abs(x.astype(np.float64))
    want = np.empty(x.size, np.uint8)
    for i, ai in enumerate(a):
        if ai >= 448:
            c = 0x7E
        else:
            d = np.abs(pos - ai)
            best = np.flatnonzero(d == d.min())
            c = best[0] if len(best) == 1 else (best[0] if best[0] % 2 == 0 else best[1])
        want[i] = c | (0x80 if np.signbit(x[i]) else 0)
    np.testing.assert_array_equal(got, want)


def test_int_casts_truncate_and_saturate():
    x = np.array([1.9, -1.9, 300.5, -300.5, np.nan, 1e20, -1e20, 2.5], np.float32)
    np.testing.assert_array_equal(cast_bits(x, DType.F32, DType.I32),
                                  [1, -1, 300, -300, 0, 2 ** 31 - 1, -2 ** 31, 2])
    np.testing.assert_array_equal(cast_bits(x, DType.F32, DType.U8), [1, 0, 255, 0, 0, 255, 0, 2])
    u = np.array(KA["u16_cast_round_trip"]["x"], np.uint16)
    np.testing.assert_array_equal(cast_bits(cast_bits(u, DType.U16, DType.F32), DType.F32, DType.U16), u)


# ---------------- known answers of the interpreter ----------------

def test_unary_known_answers():
    g = Graph()
    y = g.exp2(const(g, KA["exp2"]["x"]))
    np.testing.assert_array_equal(run(g, y).numpy(), KA["exp2"]["y"])
    s = g.sqrt(const(g, KA["sqrt"]["x"]))
    np.testing.assert_array_equal(run(g, s).numpy(), KA["sqrt"]["y"])


def test_reduce_argmax_pad_expand_known_answers():
    g = Graph()
    np.testing.assert_array_equal(run(g, g.reduce_max(const(g, KA["reduce_max"]["x"]), 1)).numpy(), KA["reduce_max"]["y"])
    np.testing.assert_array_equal(run(g, g.argmax(const(g, KA["argmax"]["x"]), 1)).numpy(), KA["argmax"]["y"])
    np.testing.assert_array_equal(run(g, g.pad(const(g, KA["pad"]["x"]), KA["pad"]["pads"])).numpy(), KA["pad"]["y"])
    np.testing.assert_array_equal(run(g, g.expand(const(g, KA["expand"]["x"]), KA["expand"]["shape"])).numpy(),
                                  KA["expand"]["y"])


def test_dot_general_known_answers():
    g = Graph()
    d = KA["dot_general_2d"]
    np.testing.assert_array_equal(run(g, g.dot_general(const(g, d["a"]), const(g, d["b"]), [1], [0])).numpy(), d["y"])
    d = KA["dot_general_batched"]
    y = g.dot_general(const(g, d["a"]), const(g, d["b"]), d["lc"], d["rc"], d["lb"], d["rb"])
    np.testing.assert_array_equal(run(g, y).numpy(), d["y"])
    d = KA["mlp_relu"]
    xw = g.dot_general(const(g, d["x"]), const(g, d["w"]), [1], [0])
    b = g.expand(g.reshape(const(g, d["b"]), [1, 4]), [2, 4])
    y = g.max(g.add(xw, b), const(g, np.zeros((2, 4))))
    np.testing.assert_array_equal(run(g, y).numpy(), d["y"])
    d = KA["golden_graph_v2"]
    y = g.sum(g.add(const(g, d["x"]), const(g, d["w"])), 1)
    np.testing.assert_array_equal(run(g, y).numpy(), d["y"])


def test_softmax_known_answer():
    g = Graph()
    x = np.array(KA["softmax_rows"]["x"], np.float32)
    y = run(g, g.softmax(const(g, x), 1)).numpy()
    e = np.exp(x - x.max(1, keepdims=True))
    assert_close(y, e / e.sum(1, keepdims=True), rtol=0, atol=KA["softmax_rows"]["tol"])


def test_low_precision_known_answers():
    g = Graph()
    d = KA["f16_add"]
    y = g.add(const(g, d["a"], DType.F16), const(g, d["b"], DType.F16))
    np.testing.assert_array_equal(to_f32(run(g, y)), d["y"])
    d = KA["bf16_identity_dot"]
    a = const(g, d["a"], DType.BF16)
    i = const(g, np.eye(2), DType.BF16)
    np.testing.assert_array_equal(to_f32(run(g, g.dot_general(a, i, [1], [0]))), d["y"])
    k = KA["f16_matmul_accumulates_in_f32"]["k"]
    y = g.dot_general(const(g, np.ones((1, k)), DType.F16), const(g, np.ones((k, 1)), DType.F16), [1], [0])
    assert to_f32(run(g, y))[0, 0] == KA["f16_matmul_accumulates_in_f32"]["y"]
    d = KA["fp8_add"]
    s = g.cast(g.add(const(g, d["a"], DType.F8E4M3), const(g, d["b"], DType.F8E4M3)), DType.F32)
    np.testing.assert_array_equal(run(g, s).numpy(), d["y"])
    d = KA["fp8_dot"]
    dd = g.cast(g.dot_general(const(g, d["a"], DType.F8E4M3), const(g, d["b"], DType.F8E4M3), [0], [0]), DType.F32)
    assert abs(run(g, dd).numpy()[()] - d["y"]) < d["tol"]
    d = KA["fp8_sqrt"]
    r = g.cast(g.sqrt(const(g, d["x"], DType.F8E4M3)), DType.F32)
    assert abs(run(g, r).numpy()[0] - d["y"][0]) < d["tol"]


def test_sdpa_known_answers():
    d = KA["sdpa_causal_first_query"]
    s, dh = d["s"], d["dh"]
    g = Graph()
    q = const(g, (np.arange(s * dh) * 0.1).reshape(s, dh))
    k = const(g, np.sin(np.arange(s * dh, dtype=np.float32) * np.float32(0.2)).reshape(s, dh))
    v = const(g, (np.arange(s * dh) + 1.0).reshape(s, dh))
    o = run(g, g.sdpa(q, k, v, True)).numpy()
    assert_close(o[0], 1.0 + np.arange(dh), rtol=0, atol=1e-5)
    d = KA["sdpa_fused_matches_decomposed"]
    b, h, s, dh = d["b"], d["h"], d["s"], d["dh"]
    n = b * h * s * dh
    mk = lambda seed: (np.sin(np.arange(n, dtype=np.float32) * np.float32(seed)) * np.float32(0.5)).reshape(b, h, s, dh)
    for causal in (False, True):
        g = Graph()
        q, k, v = const(g, mk(0.7)), const(g, mk(1.3)), const(g, mk(2.1))
        f = run(g, g.sdpa_fused(q, k, v, causal)).numpy()
        de = run(g, g.sdpa_decomposed(q, k, v, causal)).numpy()
        assert_close(f, de, rtol=0, atol=d["tol"], what=f"sdpa causal={causal}")


# ---------------- independent checks on random inputs ----------------

def test_oracle_matches_numpy_on_random_chains():
    rng = np.random.default_rng(3)
    x = rng.normal(size=(7, 33)).astype(np.float32)
    w = rng.normal(size=(33, 5)).astype(np.float32)
    g = Graph()
    xn = g.input([7, 33], DType.F32)
    wn = g.input([33, 5], DType.F32)
    feeds = {xn: Tensor.from_numpy(x), wn: Tensor.from_numpy(w)}
    outs = [g.sum(g.mul(xn, xn), 1), g.reduce_max(xn, 0), g.matmul(xn, wn), g.softmax(xn, 1),
            g.rmsnorm(xn, 1, 1e-5), g.argmax(xn, 0), g.mean(xn, 1)]
    got = interpret(g, outs, feeds)
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(1, keepdims=True))
    want = [(x64 * x64).sum(1), x.max(0), x64 @ w, e / e.sum(1, keepdims=True),
            x64 / np.sqrt((x64 * x64).mean(1, keepdims=True) + 1e-5), x.argmax(0), x64.mean(1)]
    for i, (gv, wv) in enumerate(zip(got, want)):
        if i == 5:
            np.testing.assert_array_equal(gv.numpy(), wv)
        else:
            assert_close(gv.numpy(), wv, rtol=2e-6, atol=2e-6, what=f"chain {i}")


def test_integer_semantics_match_numpy_wrapping():
    rng = np.random.default_rng(4)
    a = rng.integers(-2 ** 31, 2 ** 31, 500, dtype=np.int64).astype(np.int32)
    b = rng.integers(-2 ** 31, 2 ** 31, 500, dtype=np.int64).astype(np.int32)
    g = Graph()
    an, bn = g.input([500], DType.I32), g.input([500], DType.I32)
    feeds = {an: Tensor.from_numpy(a), bn: Tensor.from_numpy(b)}
    got = interpret(g, [g.add(an, bn), g.mul(an, bn), g.neg(an), g.sum(g.reshape(an, [5, 100]), 1)], feeds)
    with np.errstate(over="ignore"):
        np.testing.assert_array_equal(got[0].numpy(), a + b)
        np.testing.assert_array_equal(got[1].numpy(), a * b)
        np.testing.assert_array_equal(got[2].numpy(), -a)
        np.testing.assert_array_equal(got[3].numpy(), a.reshape(5, 100).sum(1, dtype=np.int32))


def test_argmax_brute_force_ties_and_nans():
    rng = np.random.default_rng(6)
    x = rng.integers(0, 4, size=(300, 9)).astype(np.float32)
    x[::7, 0] = np.nan
    x[3::11, 4] = np.nan
    g = Graph()
    xn = g.input(list(x.shape), DType.F32)
    got = run(g, g.argmax(xn, 1), {xn: Tensor.from_numpy(x)}).numpy()
    want = []
    for row in x:  # interp/reduce.rs:46-64, literally
        best, bi = row[0], 0
        for k in range(1, len(row)):
            if row[k] > best:
                best, bi = row[k], k
        want.append(bi)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("seed", range(25))
def test_realize_bit_identical_to_interpret(seed):
    # the reference's 200-graph differential fuzz (realize/fuzz.rs:114-128), smaller
    rng = np.random.default_rng(seed)
    shape = [int(rng.integers(1, 6)), int(rng.integers(1, 40))]
    g = Graph()
    x = g.input(shape, DType.F32)
    y = g.input(shape, DType.F32)
    cur = x
    for _ in range(int(rng.integers(2, 9))):
        op = rng.integers(0, 8)
        if op == 0:
            cur = g.add(cur, y)
        elif op == 1:
            cur = g.mul(cur, g.scalar(cur, float(rng.normal())))
        elif op == 2:
            cur = g.max(cur, g.neg(cur))
        elif op == 3:
            cur = g.exp2(g.mul(cur, g.scalar(cur, 0.1)))
        elif op == 4:
            cur = g.sin(cur)
        elif op == 5:
            cur = g.transpose(g.transpose(cur, 0, 1), 0, 1)
        elif op == 6:
            cur = g.sqrt(g.add(g.mul(cur, cur), g.scalar(cur, 1.0)))
        else:
            cur = g.mul(cur, g.recip(g.add(g.max(cur, g.neg(cur)), g.scalar(cur, 1.0))))
    out = g.sum(cur, 1) if rng.integers(0, 2) else cur
    feeds = {x: Tensor.from_numpy(rng.normal(size=shape).astype(np.float32)),
             y: Tensor.from_numpy(rng.normal(size=shape).astype(np.float32))}
    want = interpret(g, [out], feeds)[0].numpy()
    got, passes = realize(g, out, feeds)
    assert passes is not None
    np.testing.assert_array_equal(got.numpy(), want)


def test_realize_falls_back_off_the_f32_path():
    g = Graph()
    x = g.input([4], DType.F32)
    a = g.argmax(g.reshape(x, [2, 2]), 1)
    xv = np.array([1, 3, 2, 0], np.float32)
    got, passes = realize(g, a, {x: Tensor.from_numpy(xv)})
    assert passes is None
    np.testing.assert_array_equal(got.numpy(), [1, 0])


def test_realize_cfg1_is_two_passes():
    # realize/sched.rs:74-78: the fused elementwise producer materialises once, then reduce_v
    g = Graph()
    x = g.input([8, 64], DType.F32)
    b = g.input([64], DType.F32)
    y = g.sum(g.mul(g.relu(g.add(g.mul(x, x), g.broadcast_to(b, [8, 64]))), g.scalar(x, 0.5)), 1)
    feeds = {x: Tensor.from_numpy(np.ones((8, 64), np.float32)), b: Tensor.from_numpy(np.ones(64, np.float32))}
    got, passes = realize(g, y, feeds)
    assert passes == 2
    np.testing.assert_array_equal(got.numpy(), np.full(8, 64.0, np.float32))


def test_arg_reduce_over_an_empty_axis_is_an_error():
    """interp/reduce.rs:46 reads element 0 of the reduced axis first; with an empty axis and a
    non-empty output that is out of bounds (the reference panics): the oracle raises."""
    g = Graph()
    x = g.input([3, 0], DType.F32)
    y = g.argmax(x, 1)
    with pytest.raises(RuntimeError, match="empty axis"):
        interpret(g, [y], {x: Tensor.from_numpy(np.zeros((3, 0), np.float32))})
    # sum / max over an empty axis give the identities, like the reference's folds
    s = interpret(g, [g.sum(x, 1), g.reduce_max(x, 1)], {x: Tensor.from_numpy(np.zeros((3, 0), np.float32))})
    np.testing.assert_array_equal(s[0].numpy(), [0, 0, 0])
    np.testing.assert_array_equal(s[1].numpy(), [-np.inf] * 3)
