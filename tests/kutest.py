"""Shared test helpers: the oracle binding (test infrastructure), seeded inputs, tolerances.

The oracle (oracle/liboracle_kurumi.so) is a CPU restatement of kurumi's interpreter. Tests use
it only as the checker; the product path is kurumi_amd (libkurumi_hip.so).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

import kurumi_amd as K
from kurumi_amd import DType, Graph, Tensor

ROOT = Path(__file__).resolve().parent.parent
_ORACLE = None


def oracle() -> C.CDLL:
    global _ORACLE
    if _ORACLE is None:
        K.lib()  # the oracle resolves the IR handle symbols from the product library
        path = ROOT / "oracle" / "liboracle_kurumi.so"
        if not path.exists():
            raise RuntimeError(f"{path} not built; run `python oracle/build.py`")
        L = C.CDLL(str(path))
        P = C.c_void_p
        L.kuo_last_error.restype = C.c_char_p
        L.kuo_interpret.argtypes = [P, C.POINTER(C.c_uint32), C.c_size_t, P, C.POINTER(P)]
        L.kuo_interpret.restype = C.c_int32
        L.kuo_realize.argtypes = [P, C.c_uint32, P, C.POINTER(P), C.POINTER(C.c_int32)]
        L.kuo_realize.restype = C.c_int32
        L.kuo_threefry2x32.argtypes = [C.c_uint64, C.c_uint64]
        L.kuo_threefry2x32.restype = C.c_uint64
        L.kuo_rand_uniform.argtypes = [C.c_uint64, C.c_size_t, C.POINTER(C.c_float)]
        L.kuo_rand_uniform.restype = None
        L.kuo_cast.argtypes = [C.c_uint32, C.c_uint32, C.c_char_p, C.c_size_t, C.c_char_p]
        L.kuo_cast.restype = C.c_int32
        _ORACLE = L
    return _ORACLE


def interpret(g: Graph, roots, feeds: dict | None = None) -> list[Tensor]:
    """kurumi's reference interpreter (restated): interpret_many over `roots`."""
    roots = list(roots)
    f = K.Feeds(feeds or {})
    arr = (C.c_uint32 * len(roots))(*roots)
    out = (C.c_void_p * len(roots))()
    if oracle().kuo_interpret(g.h, arr, len(roots), f.h, out) != 0:
        raise RuntimeError("oracle: " + oracle().kuo_last_error().decode())
    return [Tensor._from_handle(out[i]) for i in range(len(roots))]


def interpret_raw(g: Graph, roots, f: "K.Feeds") -> list[int]:
    """The oracle interpreter alone, for timing: feeds bound beforehand (`K.Feeds`), outputs left
    as handles in the oracle's memory (no copy out); release them with `free_raw`."""
    roots = list(roots)
    arr = (C.c_uint32 * len(roots))(*roots)
    out = (C.c_void_p * len(roots))()
    if oracle().kuo_interpret(g.h, arr, len(roots), f.h, out) != 0:
        raise RuntimeError("oracle: " + oracle().kuo_last_error().decode())
    return [out[i] for i in range(len(roots))]


def realize_raw(g: Graph, root: int, f: "K.Feeds") -> list[int]:
    """The view-fused evaluator alone, for timing (see `interpret_raw`)."""
    out = C.c_void_p()
    passes = C.c_int32()
    if oracle().kuo_realize(g.h, root, f.h, C.byref(out), C.byref(passes)) < 0:
        raise RuntimeError("oracle: " + oracle().kuo_last_error().decode())
    return [out.value]


def free_raw(handles: list[int]) -> None:
    for h in handles:
        K.lib().ku_tensor_free(h)


def realize(g: Graph, root: int, feeds: dict | None = None) -> tuple[Tensor, int | None]:
    """View-fused CPU evaluator (restated realize::force); passes is None when it fell back."""
    f = K.Feeds(feeds or {})
    out = C.c_void_p()
    passes = C.c_int32()
    r = oracle().kuo_realize(g.h, root, f.h, C.byref(out), C.byref(passes))
    if r < 0:
        raise RuntimeError("oracle: " + oracle().kuo_last_error().decode())
    return Tensor._from_handle(out.value), (passes.value if r == 1 else None)


def cast_bits(src: np.ndarray, frm: DType, to: DType) -> np.ndarray:
    src = np.ascontiguousarray(src.astype(frm.storage, copy=False))
    n = src.size
    dst = np.empty(n, dtype=to.storage)
    buf = C.create_string_buffer(max(n * to.width, 1))
    if oracle().kuo_cast(int(frm), int(to), src.tobytes(), n, buf) != 0:
        raise RuntimeError(oracle().kuo_last_error().decode())
    return np.frombuffer(buf.raw[: n * to.width], dtype=to.storage).reshape(src.shape).copy()


def rand_uniform(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    oracle().kuo_rand_uniform(seed, n, out.ctypes.data_as(C.POINTER(C.c_float)))
    return out


def graph_values(build, shape, seed: int) -> np.ndarray:
    """Evaluate a reference random builder (e.g. Graph.randn) on the oracle: exact reference bits."""
    g = Graph()
    n = build(g, shape, seed)
    return interpret(g, [n])[0].numpy()


def randn(shape, seed: int, std: float = 1.0) -> np.ndarray:
    """kurumi `randn` (Box-Muller over threefry, graph/ops/core/random.rs:28-40) times std, f32."""
    x = graph_values(lambda g, s, sd: g.randn(s, sd), list(shape), seed)
    return (x * np.float32(std)).astype(np.float32)


def rand_range(shape, seed: int, lo: float, hi: float) -> np.ndarray:
    return graph_values(lambda g, s, sd: g.rand_range(s, sd, lo, hi), list(shape), seed)


# ---------------- bf16 helpers (numpy, test-side) ----------------

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round f32 to bf16 (nearest even) -> uint16 bits."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_f32(t: Tensor) -> np.ndarray:
    """Decode a tensor's values to f32/f64 numpy (bf16/f16/f8 decoded)."""
    a = t.numpy()
    if t.dtype == DType.BF16:
        return bf16_bits_to_f32(a)
    if t.dtype == DType.F16:
        return a.view(np.float16).astype(np.float32)
    if t.dtype in (DType.F8E4M3, DType.F8E5M2):
        return cast_bits(a, t.dtype, DType.F32)
    return a


def assert_close(got: np.ndarray, want: np.ndarray, rtol: float, atol: float, what: str = "") -> None:
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    both_nan = np.isnan(got) & np.isnan(want)
    same_inf = np.isinf(got) & np.isinf(want) & (np.sign(got) == np.sign(want))
    err = np.abs(got - want)
    ok = (err <= atol + rtol * np.abs(want)) | both_nan | same_inf
    if not ok.all():
        i = np.argmax(~ok.reshape(-1))
        a = np.broadcast_to(np.asarray(atol, dtype=np.float64), got.shape).reshape(-1)[i]
        raise AssertionError(f"{what}: {int((~ok).sum())} elements out of tolerance (rtol={rtol}, atol at that "
                             f"element={a!r}); first at {np.unravel_index(i, got.shape)}: got {got.reshape(-1)[i]!r} "
                             f"want {want.reshape(-1)[i]!r}")


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    """Spacing of bf16 values at each |x| (8 significant bits): 2^(e-7) for |x| in [2^e, 2^(e+1)),
    2^-133 below the smallest normal. Used as a per-element absolute floor for bf16 outputs."""
    a = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return np.exp2(e - 7)


def rel_err(got: np.ndarray, want: np.ndarray) -> float:
    """Normwise relative error ||got - want||_max / ||want||_max."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))
