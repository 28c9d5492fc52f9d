"""Backends in several threads of one process (the documented use: one backend per thread, all on
one GPU). Each thread builds its own backend and graphs and checks every result it gets, while
the others run; the library's process-wide state (graph ids, payload-hash memo, code-object disk
cache, the no-allocation scratch table) is shared by all of them.
"""
import threading

import numpy as np
import pytest

import kurumi_amd as K
from kurumi_amd import DType, Graph

NTHREADS = 4
ROUNDS = 12


def _fused_reduce(n):
    g = Graph()
    x = g.input([n, n], DType.F32)
    b = g.input([n], DType.F32)
    y = g.sum(g.mul(g.relu(g.add(g.mul(x, x), g.broadcast_to(b, [n, n]))), g.scalar(x, 0.5)), 1)
    return g, x, b, y


def _softmax_argmax(rows, cols):
    g = Graph()
    x = g.input([rows, cols], DType.F32)
    y = g.softmax(x, 1)
    return g, x, [y, g.cast(g.argmax(y, 1), DType.I32)]


@pytest.mark.gpu
def test_backends_in_threads_each_get_their_own_results():
    errors = []
    start = threading.Barrier(NTHREADS)

    def worker(tid):
        try:
            be = K.HipBackend()
            rng = np.random.default_rng(1000 + tid)
            n = 512 + 64 * tid  # a different kernel shape per thread as well
            g1, x1, b1, y1 = _fused_reduce(n)
            g2, x2, outs2 = _softmax_argmax(256, 1000 + 8 * tid)
            start.wait()
            for r in range(ROUNDS):
                xv = rng.uniform(-1, 1, (n, n)).astype(np.float32)
                bv = rng.uniform(-1, 1, n).astype(np.float32)
                got = be.eval_with(g1, y1, {x1: K.Tensor.from_numpy(xv), b1: K.Tensor.from_numpy(bv)}).numpy()
                want = (np.maximum(xv.astype(np.float64) ** 2 + bv, 0) * 0.5).sum(axis=1)
                np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-3,
                                           err_msg=f"thread {tid} round {r} fused reduce")
                lv = (rng.standard_normal((256, 1000 + 8 * tid)) * 3).astype(np.float32)
                sm, am = be.eval_many_with(g2, outs2, {x2: K.Tensor.from_numpy(lv)})
                sm, am = sm.numpy(), am.numpy()
                e = np.exp(lv.astype(np.float64) - lv.max(axis=1, keepdims=True))
                np.testing.assert_allclose(sm, e / e.sum(axis=1, keepdims=True), rtol=1e-4, atol=1e-7,
                                           err_msg=f"thread {tid} round {r} softmax")
                assert np.array_equal(am, sm.argmax(axis=1).astype(np.int32)), f"thread {tid} round {r} argmax"
        except Exception as ex:  # noqa: BLE001 - reported by the main thread
            errors.append(f"thread {tid}: {ex!r}")

    threads = [threading.Thread(target=worker, args=(t,), daemon=True) for t in range(NTHREADS)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a worker did not finish"
    assert not errors, errors
