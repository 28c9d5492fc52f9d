"""Device-vs-oracle differential fuzz over seeded random graphs (tests/fuzzgraphs.py).

Per-op tests pin one kernel at a time; random compositions of elementwise ops, casts,
movement through computed values, reductions, softmax and contractions make sure no
fusion/lowering combination hides between them (the reference runs the same kind of check for
its Metal backend, kurumi_metal/src/tests/fuzz.rs:183-225). Integer graphs must match the
oracle bit for bit; float graphs within fuzzgraphs.close_float, attention outputs within the
attention bar (norm-wise 1e-2 for 16-bit floats, 1e-5 for f32, and elementwise with a floor of
that size times the output's largest magnitude). The seed counts are the reference's: 40 float
graphs per float dtype, 24 integer graphs per integer dtype (fuzz.rs:195-225), run in chunks of
8 seeds per test so each test stays short; each case prints its seed before it runs and the
run stops at the first mismatch."""
import numpy as np
import pytest

import fuzzgraphs as fz
from kurumi_amd import DType
from kutest import assert_close, interpret, rel_err, to_f32

FLOAT_SEEDS, INT_SEEDS, CHUNK = 40, 24, 8


@pytest.mark.parametrize("dt", fz.FLOATS)
def test_codegen_of_random_float_graphs_compiles(dt):
    """CPU: every region kernel of a few random graphs compiles for gfx950 (hipRTC)."""
    for seed in range(2):
        g, roots = fz.float_graph(seed, dt)
        assert g.codegen(roots, compile=True) is not None


@pytest.mark.gpu
@pytest.mark.parametrize("first", range(0, FLOAT_SEEDS, CHUNK))
@pytest.mark.parametrize("dt", fz.FLOATS)
def test_random_float_graphs_match_oracle(hip, dt, first):
    for seed in range(first, first + CHUNK):
        g, roots, attn = fz.float_graph_info(seed, dt)
        print(f"fuzz {dt.name} seed {seed}: {len(roots)} roots ({len(attn)} attention)", flush=True)
        got = hip.eval_many_with(g, roots, {})
        want = interpret(g, roots)
        for i, (a, b) in enumerate(zip(got, want)):
            assert a.shape == b.shape and a.dtype == b.dtype, (seed, i, a.shape, b.shape, a.dtype, b.dtype)
            if roots[i] in attn:
                tol = 1e-5 if dt == DType.F32 else 1e-2
                gf, wf = to_f32(a), to_f32(b)
                assert rel_err(gf, wf) <= tol, (dt.name, seed, i, rel_err(gf, wf))
                assert_close(gf, wf, rtol=tol, atol=tol * np.abs(wf).max(), what=f"{dt.name} seed {seed} attention")
                continue
            ok = fz.close_float(to_f32(a), to_f32(b), b.dtype)
            if not ok.all():
                j = int(np.argmax(~ok.reshape(-1)))
                raise AssertionError(f"{dt.name} seed {seed} root {i}: {int((~ok).sum())} of {ok.size} differ; "
                                     f"first {to_f32(a).reshape(-1)[j]!r} vs {to_f32(b).reshape(-1)[j]!r}\n"
                                     + g.dump(roots[i]))


@pytest.mark.gpu
@pytest.mark.parametrize("first", range(0, INT_SEEDS, CHUNK))
@pytest.mark.parametrize("dt", fz.INTS)
def test_random_int_graphs_match_oracle_bit_exact(hip, dt, first):
    for seed in range(first, first + CHUNK):
        g, roots = fz.int_graph(seed, dt)
        print(f"fuzz {dt.name} seed {seed}: {len(roots)} roots", flush=True)
        got = hip.eval_many_with(g, roots, {})
        want = interpret(g, roots)
        for i, (a, b) in enumerate(zip(got, want)):
            assert a.shape == b.shape and a.dtype == b.dtype, (seed, i)
            np.testing.assert_array_equal(a.numpy(), b.numpy(), err_msg=f"{dt.name} seed {seed} root {i}\n"
                                          + g.dump(roots[i]))
