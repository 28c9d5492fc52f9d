"""C-ABI contract of libkurumi_hip.so on the CPU (no GPU calls): every declared symbol is
exported, record-time errors surface as KU_ERR + ku_last_error, handles are null-safe, and
backend creation fails cleanly (NULL + message) without a device — mirroring the reference's
ABI tests (kurumi/src/capi/tests.rs:32-278, capi/tests/drift.rs:1-60)."""
import ctypes as C
import os
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import kurumi_amd as K
from kurumi_amd import DType, Graph, Tensor

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "kurumi_hip.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ku_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    L = K.lib()
    syms = declared_symbols()
    assert len(syms) > 90
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing


def test_exports_are_declared():
    # drift guard the other way: every exported ku_* symbol is in the header
    out = subprocess.run(["nm", "-D", "--defined-only", str(ROOT / "kurumi_amd" / "libkurumi_hip.so")],
                         capture_output=True, text=True).stdout
    exported = sorted({m for m in re.findall(r"\bT (ku_[a-z0-9_]+)$", out, flags=re.M)})
    assert set(exported) <= set(declared_symbols()), sorted(set(exported) - set(declared_symbols()))


def test_builder_errors_return_ku_err_with_message():
    L = K.lib()
    g = L.ku_graph_new()
    shp = (C.c_size_t * 2)(2, 3)
    a = L.ku_input(g, shp, 2, int(DType.F32))
    shp2 = (C.c_size_t * 2)(3, 2)
    b = L.ku_input(g, shp2, 2, int(DType.F32))
    assert L.ku_add(g, a, b) == K.KU_ERR
    assert b"add" in L.ku_last_error() and b"[2, 3]" in L.ku_last_error()
    c = L.ku_input(g, shp, 2, int(DType.I32))
    assert L.ku_mul(g, a, c) == K.KU_ERR
    assert b"dtype" in L.ku_last_error()
    assert L.ku_sum(g, a, 5) == K.KU_ERR and b"out of range" in L.ku_last_error()
    assert L.ku_neg(g, 999) == K.KU_ERR
    assert L.ku_input(None, shp, 2, 13) == K.KU_ERR and b"null graph" in L.ku_last_error()
    assert L.ku_cast(g, a, 99) == K.KU_ERR and b"dtype" in L.ku_last_error()
    L.ku_graph_free(g)


def test_python_builders_raise_on_record_time_errors():
    g = Graph()
    x = g.input([2, 3], DType.F32)
    with pytest.raises(K.KuError, match="reshape"):
        g.reshape(x, [4, 2])
    with pytest.raises(K.KuError, match="expand"):
        g.expand(x, [3, 3])
    with pytest.raises(K.KuError, match="dot_general"):
        g.dot_general(x, x, [1], [1], [0], [1])
    with pytest.raises(K.KuError, match="softmax"):
        g.softmax(g.input([2], DType.I32), 0)


def test_null_handles_are_safe():
    L = K.lib()
    assert not L.ku_eval(None, 0, None)
    assert b"null" in L.ku_last_error()
    assert not L.ku_eval_with(None, 0, None, None)
    out = (C.c_void_p * 1)()
    assert L.ku_eval_many(None, None, 0, None, None, out) == -1
    assert L.ku_node_rank(None, 0) == C.c_size_t(-1).value
    assert L.ku_node_dtype(None, 0) == K.KU_ERR
    assert not L.ku_plan_compile(None, 0)
    assert not L.ku_plan_run(None, None, None)
    L.ku_graph_free(None)
    L.ku_tensor_free(None)
    L.ku_feeds_free(None)
    L.ku_backend_free(None)
    L.ku_plan_free(None)
    L.ku_hip_plan_free(None)


def test_backend_kinds():
    L = K.lib()
    assert not L.ku_backend_new(0)
    assert b"CPU backend" in L.ku_last_error()
    assert not L.ku_backend_new(1)
    assert b"Metal" in L.ku_last_error()
    assert not L.ku_backend_new(7)
    assert b"unknown kind" in L.ku_last_error()


def test_hip_backend_absent_device_is_null_with_message():
    # forced from the host so it behaves the same on a GPU box
    code = ("import os, sys; sys.path.insert(0, %r); os.environ['KURUMI_HIP_FORCE_NO_DEVICE'] = '1'; "
            "import kurumi_amd as K; h = K.lib().ku_backend_new(2); "
            "print('NULL' if not h else 'HANDLE', K.lib().ku_last_error().decode())") % str(ROOT)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.stdout.startswith("NULL"), r.stdout + r.stderr
    assert "no HIP device" in r.stdout


def test_inspection_shape_dtype_dump_count():
    g = Graph()
    x = g.input([2, 3], DType.BF16)
    y = g.sum(g.mul(x, x), 1)
    a = g.argmax(x, 0)
    assert g.shape(y) == (2,) and g.dtype(y) == DType.BF16
    assert g.shape(a) == (3,) and g.dtype(a) == DType.I64
    d = g.dump(y)
    assert d.splitlines() == ["%0 = Input[2, 3]() : [2, 3]", "%1 = Mul(%0, %0) : [2, 3]",
                              "%2 = Sum { axis: 1 }(%1) : [2]"]
    assert g.node_count(y) == 3
    dg = g.dot_general(g.input([4, 2, 5], DType.F32), g.input([4, 5, 7], DType.F32), [2], [1], [0], [0])
    assert g.shape(dg) == (4, 2, 7)
    s = g.sdpa(g.input([1, 2, 8, 4], DType.F32), g.input([1, 2, 8, 4], DType.F32), g.input([1, 2, 8, 4], DType.F32),
               True)
    assert g.shape(s) == (1, 2, 8, 4)


def test_sdpa_selects_fused_above_one_gib_like_the_reference():
    # graph/ops/nn/attention.rs:83-90: the [..,S,S] f32 score buffer decides
    g = Graph()
    big = [4, 32, 2048, 128]
    q, k, v = (g.input(big, DType.BF16) for _ in range(3))
    assert "Sdpa { causal: true }" in g.dump(g.sdpa(q, k, v, True)).splitlines()[-1]
    small = [2, 4, 64, 32]
    q, k, v = (g.input(small, DType.BF16) for _ in range(3))
    assert "DotGeneral" in g.dump(g.sdpa(q, k, v, True)).splitlines()[-1]


def test_tensor_round_trip_and_f32_readout():
    L = K.lib()
    x = np.arange(6, dtype=np.float32).reshape(2, 3)
    t = Tensor.from_numpy(x)
    h = t._handle()
    assert L.ku_tensor_rank(h) == 2 and L.ku_tensor_len(h) == 6 and L.ku_tensor_dtype(h) == int(DType.F32)
    buf = (C.c_float * 6)()
    assert L.ku_tensor_data_f32(h, buf, 6) == 6
    np.testing.assert_array_equal(np.frombuffer(buf, np.float32), x.ravel())
    assert L.ku_tensor_data_f32(h, buf, 2) == -1
    back = Tensor._from_handle(h)
    np.testing.assert_array_equal(back.numpy(), x)
    bad = L.ku_tensor_new(int(DType.F32), b"\x00" * 5, 5, (C.c_size_t * 1)(2), 1)
    assert not bad and b"nbytes" in L.ku_last_error()


@pytest.mark.parametrize("nbytes", [(16 << 20) + 4 * 12345, (40 << 20) - 4 * 7, 4 * 8 * 3])
def test_large_tensor_round_trip_is_bit_exact(nbytes):
    # ku_tensor_new / ku_tensor_bytes split copies of 16 MiB and more across threads on page
    # boundaries; every byte must land in place for ragged sizes too (and the small case stays
    # on one memcpy)
    n = nbytes // 4
    x = np.random.default_rng(nbytes).integers(0, 2**32, n, dtype=np.uint32).view(np.float32)
    t = Tensor(DType.F32, [n], x.tobytes())
    back = Tensor._from_handle(t._handle())
    assert isinstance(back.data, np.ndarray) and back.data.nbytes == nbytes
    np.testing.assert_array_equal(back.numpy().view(np.uint32), x.view(np.uint32))
    # a numpy-backed tensor feeds the C side as well as a bytes-backed one
    again = Tensor._from_handle(back._handle())
    np.testing.assert_array_equal(again.numpy().view(np.uint32), x.view(np.uint32))
    buf = np.empty(n, np.float32)
    h = back._handle()
    assert K.lib().ku_tensor_data_f32(h, buf.ctypes.data_as(C.POINTER(C.c_float)), n) == n
    K.lib().ku_tensor_free(h)
    np.testing.assert_array_equal(buf.view(np.uint32), x.view(np.uint32))


def test_scalar_constant_takes_the_tensor_dtype():
    # elementwise.rs:83-94: the scalar const is built directly in like's dtype
    g = Graph()
    x = g.input([3], DType.BF16)
    s = g.scalar(x, 1.44269504)
    assert g.dtype(s) == DType.BF16 and g.shape(s) == (3,)
