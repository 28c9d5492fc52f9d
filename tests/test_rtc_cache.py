"""The hipRTC code-object cache on disk (KURUMI_HIP_CACHE): backends in several threads of one
process may compile the same kernel at once, and a damaged cached object must not break a run.

The CPU test compiles through ku_hip_codegen (hipRTC needs no GPU); the GPU test loads the
cached object through a backend's kernel loader.
"""
import threading

import numpy as np
import pytest

import kurumi_amd as K
from kurumi_amd import DType, Graph


def _graph(c: float):
    """A small fused chain whose generated source carries the constant c (so a fresh c gives a
    kernel no cache has seen)."""
    g = Graph()
    x = g.input([64, 256], DType.F32)
    y = g.sum(g.mul(g.relu(g.add(x, g.scalar(x, c))), g.scalar(x, 0.5)), 1)
    return g, x, y


def _cache_files(d):
    files = sorted(p.name for p in d.iterdir())
    return [f for f in files if f.endswith(".co")], [f for f in files if ".tmp" in f]


def test_concurrent_compiles_leave_one_whole_code_object(tmp_path, monkeypatch):
    monkeypatch.setenv("KURUMI_HIP_CACHE", str(tmp_path))
    c = 1.0 + float(np.random.default_rng().integers(1, 1 << 30)) / (1 << 31)
    errors, sources = [], []
    start = threading.Barrier(8)

    def worker():
        try:
            g, _, y = _graph(c)  # each thread its own (identical) graph
            start.wait()
            sources.append(g.codegen([y], compile=True))
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=worker) for _ in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    assert len(set(sources)) == 1
    cos, tmps = _cache_files(tmp_path)
    assert len(cos) == 1 and not tmps, (cos, tmps)
    blob = (tmp_path / cos[0]).read_bytes()
    assert blob[:4] == b"\x7fELF" and len(blob) > 1024
    # a later compile of the same source is served from that file and leaves it as it was
    g, _, y = _graph(c)
    g.codegen([y], compile=True)
    assert _cache_files(tmp_path) == (cos, []) and (tmp_path / cos[0]).read_bytes() == blob


@pytest.mark.gpu
def test_damaged_cached_code_object_is_recompiled(hip, tmp_path, monkeypatch):
    monkeypatch.setenv("KURUMI_HIP_CACHE", str(tmp_path))
    c = 1.0 + float(np.random.default_rng().integers(1, 1 << 30)) / (1 << 31)
    g, x, y = _graph(c)
    g.codegen([y], compile=True)  # puts the kernel's code object in the cache
    cos, _ = _cache_files(tmp_path)
    assert len(cos) == 1
    (tmp_path / cos[0]).write_bytes(b"not a code object " * 64)  # as a damaged file would be
    xv = np.linspace(-2.0, 2.0, 64 * 256, dtype=np.float32).reshape(64, 256)
    got = hip.eval_with(g, y, {x: K.Tensor.from_numpy(xv)}).numpy()
    want = (np.maximum(xv + np.float32(c), 0) * np.float32(0.5)).sum(axis=1, dtype=np.float64)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-4)
    blob = (tmp_path / cos[0]).read_bytes()
    assert blob[:4] == b"\x7fELF"  # the fresh compile replaced the damaged file
