"""kurumi_amd: Python mirror of the kurumi graph/backend API over libkurumi_hip.so.

The classes follow the reference's Rust surface (kurumi_core `Graph` builders,
`Backend::eval / eval_with / eval_many_with`, `TensorVal`) and go through the C ABI declared
in ``include/kurumi_hip.h``. The HIP backend is the only executor: there is no CPU fallback in
this package, and `HipBackend()` raises when no MI355X is available.
"""
from __future__ import annotations

import ctypes as C
import enum
import os
from pathlib import Path
from typing import Iterable, Sequence

import numpy as np

__all__ = ["DType", "Graph", "HipBackend", "Plan", "Tensor", "KuError", "lib", "amp", "amp_fp8", "KU_ERR"]

_PKG = Path(__file__).resolve().parent
_LIB_PATH = _PKG / "libkurumi_hip.so"
KU_ERR = 0xFFFFFFFF


class KuError(RuntimeError):
    pass


class DType(enum.IntEnum):
    BOOL = 0
    U8 = 1
    U16 = 2
    U32 = 3
    U64 = 4
    I8 = 5
    I16 = 6
    I32 = 7
    I64 = 8
    F8E4M3 = 9
    F8E5M2 = 10
    F16 = 11
    BF16 = 12
    F32 = 13
    F64 = 14
    C64 = 15
    C128 = 16

    @property
    def width(self) -> int:
        return {0: 1, 1: 1, 2: 2, 3: 4, 4: 8, 5: 1, 6: 2, 7: 4, 8: 8, 9: 1, 10: 1, 11: 2, 12: 2, 13: 4, 14: 8,
                15: 8, 16: 16}[int(self)]

    @property
    def storage(self) -> np.dtype:
        """numpy dtype of the raw little-endian storage (bf16/f16/f8 as unsigned bits)."""
        return np.dtype({0: np.uint8, 1: np.uint8, 2: np.uint16, 3: np.uint32, 4: np.uint64, 5: np.int8,
                         6: np.int16, 7: np.int32, 8: np.int64, 9: np.uint8, 10: np.uint8, 11: np.uint16,
                         12: np.uint16, 13: np.float32, 14: np.float64, 15: np.complex64,
                         16: np.complex128}[int(self)])


_lib = None


def lib() -> C.CDLL:
    """Load libkurumi_hip.so (built in-tree by ``kurumi_amd.build``); fail loudly if absent."""
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise KuError(f"{_LIB_PATH} is not built; run `python -m kurumi_amd.build`")
        _lib = C.CDLL(str(_LIB_PATH))
        _declare(_lib)
    return _lib


def _declare(L: C.CDLL) -> None:
    sz = C.c_size_t
    P = C.c_void_p
    u32 = C.c_uint32
    psz = C.POINTER(C.c_size_t)
    sig = {
        "ku_last_error": ([], C.c_char_p),
        "ku_graph_new": ([], P),
        "ku_graph_free": ([P], None),
        "ku_input": ([P, psz, sz, u32], u32),
        "ku_constant_f32": ([P, C.POINTER(C.c_float), sz, psz, sz], u32),
        "ku_constant": ([P, u32, C.c_void_p, sz, psz, sz], u32),
        "ku_scalar": ([P, u32, C.c_float], u32),
        "ku_where": ([P, u32, u32, u32], u32),
        "ku_clamp_min": ([P, u32, C.c_float], u32),
        "ku_rmsnorm": ([P, u32, sz, C.c_float], u32),
        "ku_dot_general": ([P, u32, u32, psz, sz, psz, sz, psz, sz, psz, sz], u32),
        "ku_reshape": ([P, u32, psz, sz], u32),
        "ku_expand": ([P, u32, psz, sz], u32),
        "ku_permute": ([P, u32, psz, sz], u32),
        "ku_broadcast_to": ([P, u32, psz, sz], u32),
        "ku_transpose": ([P, u32, sz, sz], u32),
        "ku_flip": ([P, u32, psz, sz], u32),
        "ku_slice": ([P, u32, psz, sz], u32),
        "ku_slice_step": ([P, u32, psz, sz], u32),
        "ku_pad": ([P, u32, psz, sz], u32),
        "ku_iota": ([P, psz, sz, sz, u32], u32),
        "ku_cast": ([P, u32, u32], u32),
        "ku_bitcast": ([P, u32, u32], u32),
        "ku_sdpa": ([P, u32, u32, u32, u32], u32),
        "ku_sdpa_decomposed": ([P, u32, u32, u32, u32], u32),
        "ku_sdpa_fused": ([P, u32, u32, u32, u32], u32),
        "ku_rand_uniform": ([P, psz, sz, C.c_uint64], u32),
        "ku_randn": ([P, psz, sz, C.c_uint64], u32),
        "ku_rand_range": ([P, psz, sz, C.c_uint64, C.c_float, C.c_float], u32),
        "ku_amp_fp8": ([P, u32], u32),
        "ku_amp": ([P, u32], u32),
        "ku_backend_new": ([u32], P),
        "ku_backend_free": ([P], None),
        "ku_eval": ([P, u32, P], P),
        "ku_eval_with": ([P, u32, P, P], P),
        "ku_eval_many": ([P, C.POINTER(C.c_uint32), sz, P, P, C.POINTER(P)], C.c_int32),
        "ku_node_count": ([P, u32], sz),
        "ku_dump": ([P, u32, C.c_char_p, sz], sz),
        "ku_node_rank": ([P, u32], sz),
        "ku_node_shape": ([P, u32, psz], None),
        "ku_node_dtype": ([P, u32], u32),
        "ku_plan_compile": ([P, u32], P),
        "ku_plan_run": ([P, P, P], P),
        "ku_plan_free": ([P], None),
        "ku_hip_plan_compile_on": ([P, P, u32], P),
        "ku_feeds_new": ([], P),
        "ku_feeds_free": ([P], None),
        "ku_feeds_set": ([P, u32, P], None),
        "ku_tensor_f32": ([C.POINTER(C.c_float), sz, psz, sz], P),
        "ku_tensor_new": ([u32, C.c_void_p, sz, psz, sz], P),
        "ku_tensor_free": ([P], None),
        "ku_tensor_rank": ([P], sz),
        "ku_tensor_shape": ([P, psz], None),
        "ku_tensor_len": ([P], sz),
        "ku_tensor_dtype": ([P], u32),
        "ku_tensor_data_f32": ([P, C.POINTER(C.c_float), sz], C.c_ssize_t),
        "ku_tensor_nbytes": ([P], sz),
        "ku_tensor_bytes": ([P, C.c_void_p], None),
        "ku_hip_plan_new": ([P, C.POINTER(C.c_uint32), sz, P, P], P),
        "ku_hip_plan_feed": ([P, u32, P], C.c_int32),
        "ku_hip_plan_launch": ([P, u32], C.c_int32),
        "ku_hip_plan_sync": ([P], C.c_int32),
        "ku_hip_plan_output": ([P, sz], P),
        "ku_hip_plan_num_steps": ([P], sz),
        "ku_hip_plan_step_label": ([P, sz, C.c_char_p, sz], sz),
        "ku_hip_plan_time_steps": ([P, C.c_int32, C.POINTER(C.c_double), sz], C.c_int32),
        "ku_hip_plan_time": ([P, C.c_int32, u32], C.c_double),
        "ku_hip_plan_free": ([P], None),
        "ku_hip_plans_time": ([C.POINTER(P), sz, C.c_int32, u32], C.c_double),
        "ku_hip_codegen": ([P, C.POINTER(C.c_uint32), sz, u32, C.c_char_p, sz], sz),
        "ku_hip_profile": ([P, C.POINTER(C.c_uint64), sz], C.c_uint64),
        "ku_hip_linear_e4m3": ([P, P, u32, P, P, P, u32, sz, sz, sz, P], C.c_int32),
        "ku_hip_linear_e4m3_noalloc": ([P, u32, P, P, P, u32, sz, sz, sz, P], C.c_int32),
        "ku_quant_matmul": ([P, u32, u32, u32, u32, C.c_uint8, sz], u32),
        "ku_quantize": ([C.POINTER(C.c_float), sz, sz, C.c_uint8, sz, u32, C.c_char_p, C.POINTER(C.c_uint16),
                         C.POINTER(C.c_uint16)], None),
        "ku_graph_serialize": ([P, C.POINTER(u32), sz, C.POINTER(u32), C.POINTER(C.c_uint8),
                                C.POINTER(C.c_char_p), sz, C.c_char_p, sz], sz),
        "ku_graph_serialize_reachable": ([P, C.POINTER(u32), sz, C.POINTER(u32), C.POINTER(C.c_uint8),
                                          C.POINTER(C.c_char_p), sz, C.c_char_p, sz], sz),
        "ku_graph_serialize_multi": ([P, sz, C.POINTER(C.c_char_p), C.POINTER(u32), C.POINTER(u32), C.POINTER(u32),
                                      C.POINTER(u32), C.POINTER(C.c_uint8), C.POINTER(C.c_char_p), C.c_char_p, sz],
                                     sz),
        "ku_graph_deserialize": ([C.c_char_p, sz], P),
        "ku_runnable_take_graph": ([P], P),
        "ku_runnable_output_count": ([P], sz),
        "ku_runnable_output": ([P, sz], u32),
        "ku_runnable_input_count": ([P], sz),
        "ku_runnable_input_node": ([P, sz], u32),
        "ku_runnable_input_role": ([P, sz], u32),
        "ku_runnable_input_name": ([P, sz, C.c_char_p, sz], sz),
        "ku_runnable_entry_count": ([P], sz),
        "ku_runnable_entry_name": ([P, sz, C.c_char_p, sz], sz),
        "ku_runnable_entry_output_count": ([P, sz], sz),
        "ku_runnable_entry_output": ([P, sz, sz], u32),
        "ku_runnable_entry_input_count": ([P, sz], sz),
        "ku_runnable_entry_input_node": ([P, sz, sz], u32),
        "ku_runnable_entry_input_role": ([P, sz, sz], u32),
        "ku_runnable_entry_input_name": ([P, sz, sz, C.c_char_p, sz], sz),
        "ku_runnable_free": ([P], None),
    }
    for name in ["ku_add", "ku_sub", "ku_mul", "ku_div", "ku_max", "ku_idiv", "ku_and", "ku_or", "ku_xor", "ku_shl",
                 "ku_shr", "ku_lt", "ku_eq", "ku_matmul"]:
        sig[name] = ([P, u32, u32], u32)
    for name in ["ku_neg", "ku_recip", "ku_sqrt", "ku_square", "ku_abs", "ku_floor", "ku_exp", "ku_exp2", "ku_ln",
                 "ku_log2", "ku_sin", "ku_cos", "ku_relu", "ku_detach", "ku_flatten", "ku_t", "ku_sum_all",
                 "ku_sigmoid", "ku_silu", "ku_tanh", "ku_gelu", "ku_rope", "ku_sign", "ku_ceil", "ku_round"]:
        sig[name] = ([P, u32], u32)
    for name in ["ku_sum", "ku_prod", "ku_mean", "ku_reduce_max", "ku_argmax", "ku_argmin", "ku_softmax",
                 "ku_squeeze", "ku_unsqueeze", "ku_reduce_min", "ku_logsumexp", "ku_log_softmax"]:
        sig[name] = ([P, u32, sz], u32)
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res


def last_error() -> str:
    e = lib().ku_last_error()
    return e.decode() if e else ""


def _shape(s: Sequence[int]):
    arr = (C.c_size_t * max(len(s), 1))(*[int(x) for x in s])
    return arr, len(s)


def _check_node(n: int, what: str) -> int:
    if n == KU_ERR:
        raise KuError(f"{what}: {last_error()}")
    return n


def _raw(data):
    """(pointer, byte length) of a tensor's storage: `bytes`/`bytearray`, or a C-contiguous
    numpy array (the storage of tensors that came back from the library)."""
    if isinstance(data, np.ndarray):
        if not data.flags.c_contiguous:
            raise KuError("tensor storage must be C-contiguous")
        return (data.ctypes.data if data.nbytes else None), data.nbytes
    if isinstance(data, bytearray):
        return (C.addressof(C.c_char.from_buffer(data)) if data else None), len(data)
    return bytes(data), len(data)


class Tensor:
    """Owned host tensor (the reference's `TensorVal`): dtype, shape, raw LE bytes.

    `data` is `bytes` for tensors built here and a flat `uint8` numpy array for tensors
    returned by the library (one copy out of the C handle instead of three); both expose the
    buffer protocol and `len()` in bytes.
    """

    def __init__(self, dtype: DType, shape: Sequence[int], data):
        self.dtype = DType(dtype)
        self.shape = tuple(int(x) for x in shape)
        self.data = data

    @staticmethod
    def from_numpy(a: np.ndarray, dtype: DType | None = None) -> "Tensor":
        if dtype is None:
            dtype = {np.dtype(np.float32): DType.F32, np.dtype(np.float64): DType.F64,
                     np.dtype(np.int32): DType.I32, np.dtype(np.int64): DType.I64, np.dtype(np.uint8): DType.U8,
                     np.dtype(np.int8): DType.I8, np.dtype(np.int16): DType.I16, np.dtype(np.uint16): DType.U16,
                     np.dtype(np.uint32): DType.U32, np.dtype(np.uint64): DType.U64,
                     np.dtype(np.bool_): DType.BOOL}[a.dtype]
        a = np.ascontiguousarray(a)
        if a.dtype == np.bool_:
            a = a.astype(np.uint8)
        if a.dtype.itemsize != DType(dtype).width:
            raise KuError(f"numpy dtype {a.dtype} does not store {DType(dtype).name}")
        return Tensor(dtype, a.shape, a.tobytes())

    def numpy(self) -> np.ndarray:
        """Raw storage as numpy (bf16/f16/f8 come back as their unsigned bit patterns)."""
        a = np.frombuffer(self.data, dtype=self.dtype.storage).reshape(self.shape)
        if self.dtype == DType.BOOL:
            return a.astype(np.bool_)
        return a.copy()

    def _handle(self):
        s, r = _shape(self.shape)
        ptr, n = _raw(self.data)
        h = lib().ku_tensor_new(int(self.dtype), ptr, n, s, r)
        if not h:
            raise KuError(f"ku_tensor_new: {last_error()}")
        return h

    @staticmethod
    def _from_handle(h) -> "Tensor":
        L = lib()
        r = L.ku_tensor_rank(h)
        shp = (C.c_size_t * max(r, 1))()
        L.ku_tensor_shape(h, shp)
        n = L.ku_tensor_nbytes(h)
        buf = np.empty(n, np.uint8)
        if n:
            L.ku_tensor_bytes(h, buf.ctypes.data)
        t = Tensor(DType(L.ku_tensor_dtype(h)), list(shp)[:r], buf)
        L.ku_tensor_free(h)
        return t


class Feeds:
    def __init__(self, feeds: dict[int, Tensor] | None = None):
        self.h = lib().ku_feeds_new()
        for k, v in (feeds or {}).items():
            th = v._handle()
            lib().ku_feeds_set(self.h, int(k), th)
            lib().ku_tensor_free(th)

    def __del__(self):
        if getattr(self, "h", None):
            lib().ku_feeds_free(self.h)
            self.h = None


class Graph:
    """Append-only graph builder (kurumi_core/src/graph.rs); methods return node ids."""

    def __init__(self, _handle=None):
        self.h = _handle if _handle else lib().ku_graph_new()

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.ku_graph_free(self.h)
            self.h = None

    def _n(self, name: str, *args) -> int:
        return _check_node(getattr(lib(), name)(self.h, *args), name)

    # leaves
    def input(self, shape: Sequence[int], dtype: DType) -> int:
        s, r = _shape(shape)
        return self._n("ku_input", s, r, int(dtype))

    def constant(self, data: np.ndarray, dtype: DType | None = None) -> int:
        t = Tensor.from_numpy(np.asarray(data), dtype)
        s, r = _shape(t.shape)
        ptr, n = _raw(t.data)
        return self._n("ku_constant", int(t.dtype), ptr, n, s, r)

    def constant_bytes(self, dtype: DType, raw, shape: Sequence[int]) -> int:
        s, r = _shape(shape)
        ptr, n = _raw(raw)
        return self._n("ku_constant", int(dtype), ptr, n, s, r)

    def scalar(self, like: int, v: float) -> int:
        return self._n("ku_scalar", like, float(v))

    def where(self, c: int, a: int, b: int) -> int:
        return self._n("ku_where", c, a, b)

    def clamp_min(self, x: int, v: float) -> int:
        return self._n("ku_clamp_min", x, float(v))

    def rmsnorm(self, x: int, axis: int, eps: float) -> int:
        return self._n("ku_rmsnorm", x, axis, float(eps))

    def dot_general(self, a: int, b: int, lc: Sequence[int], rc: Sequence[int], lb: Sequence[int] = (),
                    rb: Sequence[int] = ()) -> int:
        args = []
        for v in (lc, rc, lb, rb):
            arr, n = _shape(v)
            args += [arr, n]
        return self._n("ku_dot_general", a, b, *args)

    def quant_matmul(self, act: int, qweight: int, scales: int, mins: int | None, bits: int, group_size: int) -> int:
        """act [M, K] x dequant(qweight)[N, K]^T (graph/ops/core/contract.rs:49-115); mins None = symmetric."""
        return self._n("ku_quant_matmul", act, qweight, scales, KU_ERR if mins is None else mins, bits, group_size)

    def reshape(self, x: int, shape: Sequence[int]) -> int:
        s, r = _shape(shape)
        return self._n("ku_reshape", x, s, r)

    def expand(self, x: int, shape: Sequence[int]) -> int:
        s, r = _shape(shape)
        return self._n("ku_expand", x, s, r)

    def broadcast_to(self, x: int, shape: Sequence[int]) -> int:
        s, r = _shape(shape)
        return self._n("ku_broadcast_to", x, s, r)

    def permute(self, x: int, perm: Sequence[int]) -> int:
        s, r = _shape(perm)
        return self._n("ku_permute", x, s, r)

    def transpose(self, x: int, i: int, j: int) -> int:
        return self._n("ku_transpose", x, i, j)

    def flip(self, x: int, axes: Sequence[int]) -> int:
        s, r = _shape(axes)
        return self._n("ku_flip", x, s, r)

    def slice(self, x: int, ranges: Sequence[tuple[int, int]]) -> int:
        flat = [v for rg in ranges for v in rg]
        s, _ = _shape(flat)
        return self._n("ku_slice", x, s, len(ranges))

    def slice_step(self, x: int, ranges: Sequence[tuple[int, int, int]]) -> int:
        flat = [v for rg in ranges for v in rg]
        s, _ = _shape(flat)
        return self._n("ku_slice_step", x, s, len(ranges))

    def pad(self, x: int, pads: Sequence[tuple[int, int]]) -> int:
        flat = [v for p in pads for v in p]
        s, _ = _shape(flat)
        return self._n("ku_pad", x, s, len(pads))

    def iota(self, shape: Sequence[int], axis: int, dtype: DType) -> int:
        s, r = _shape(shape)
        return self._n("ku_iota", s, r, axis, int(dtype))

    def cast(self, x: int, dtype: DType) -> int:
        return self._n("ku_cast", x, int(dtype))

    def bitcast(self, x: int, dtype: DType) -> int:
        return self._n("ku_bitcast", x, int(dtype))

    def sdpa(self, q: int, k: int, v: int, causal: bool) -> int:
        return self._n("ku_sdpa", q, k, v, int(causal))

    def sdpa_decomposed(self, q: int, k: int, v: int, causal: bool) -> int:
        return self._n("ku_sdpa_decomposed", q, k, v, int(causal))

    def sdpa_fused(self, q: int, k: int, v: int, causal: bool) -> int:
        return self._n("ku_sdpa_fused", q, k, v, int(causal))

    def rand_uniform(self, shape: Sequence[int], seed: int) -> int:
        s, r = _shape(shape)
        return self._n("ku_rand_uniform", s, r, seed)

    def randn(self, shape: Sequence[int], seed: int) -> int:
        s, r = _shape(shape)
        return self._n("ku_randn", s, r, seed)

    def rand_range(self, shape: Sequence[int], seed: int, lo: float, hi: float) -> int:
        s, r = _shape(shape)
        return self._n("ku_rand_range", s, r, seed, lo, hi)

    # inspection
    def shape(self, n: int) -> tuple[int, ...]:
        r = lib().ku_node_rank(self.h, n)
        if r == C.c_size_t(-1).value:
            raise KuError(last_error())
        out = (C.c_size_t * max(r, 1))()
        lib().ku_node_shape(self.h, n, out)
        return tuple(out[:r])

    def dtype(self, n: int) -> DType:
        d = lib().ku_node_dtype(self.h, n)
        if d == KU_ERR:
            raise KuError(last_error())
        return DType(d)

    def node_count(self, root: int) -> int:
        return lib().ku_node_count(self.h, root)

    def dump(self, root: int) -> str:
        n = lib().ku_dump(self.h, root, None, 0)
        buf = C.create_string_buffer(n + 1)
        lib().ku_dump(self.h, root, buf, n)
        return buf.raw[:n].decode()

    def codegen(self, roots: Iterable[int], compile: bool = False) -> str:
        roots = list(roots)
        arr = (C.c_uint32 * len(roots))(*roots)
        n = lib().ku_hip_codegen(self.h, arr, len(roots), int(compile), None, 0)
        if n == 0 and last_error():
            raise KuError(last_error())
        buf = C.create_string_buffer(n + 1)
        lib().ku_hip_codegen(self.h, arr, len(roots), int(compile), buf, n)
        return buf.raw[:n].decode()


def _add_simple(name: str, cname: str, nargs: int) -> None:
    if nargs == 1:
        def f(self, x):
            return self._n(cname, x)
    elif nargs == 2:
        def f(self, a, b):
            return self._n(cname, a, b)
    else:
        def f(self, x, axis):
            return self._n(cname, x, axis)
    f.__name__ = name
    setattr(Graph, name, f)


for _n, _c in [("add", "ku_add"), ("sub", "ku_sub"), ("mul", "ku_mul"), ("div", "ku_div"), ("max", "ku_max"),
               ("idiv", "ku_idiv"), ("bit_and", "ku_and"), ("bit_or", "ku_or"), ("bit_xor", "ku_xor"),
               ("shl", "ku_shl"), ("shr", "ku_shr"), ("lt", "ku_lt"), ("eq", "ku_eq"), ("matmul", "ku_matmul")]:
    _add_simple(_n, _c, 2)
for _n, _c in [("neg", "ku_neg"), ("recip", "ku_recip"), ("sqrt", "ku_sqrt"), ("square", "ku_square"),
               ("abs", "ku_abs"), ("floor", "ku_floor"), ("exp", "ku_exp"), ("exp2", "ku_exp2"), ("ln", "ku_ln"),
               ("log2", "ku_log2"), ("sin", "ku_sin"), ("cos", "ku_cos"), ("relu", "ku_relu"),
               ("detach", "ku_detach"), ("flatten", "ku_flatten"), ("t", "ku_t"), ("sum_all", "ku_sum_all"),
               ("sigmoid", "ku_sigmoid"), ("silu", "ku_silu"), ("tanh", "ku_tanh"), ("gelu", "ku_gelu"),
               ("rope", "ku_rope"), ("sign", "ku_sign"), ("ceil", "ku_ceil"), ("round", "ku_round")]:
    _add_simple(_n, _c, 1)
for _n, _c in [("sum", "ku_sum"), ("prod", "ku_prod"), ("mean", "ku_mean"), ("reduce_max", "ku_reduce_max"),
               ("argmax", "ku_argmax"), ("argmin", "ku_argmin"), ("softmax", "ku_softmax"),
               ("squeeze", "ku_squeeze"), ("unsqueeze", "ku_unsqueeze"), ("reduce_min", "ku_reduce_min"),
               ("logsumexp", "ku_logsumexp"), ("log_softmax", "ku_log_softmax")]:
    _add_simple(_n, _c, 3)


# ---- KGPH v2 graph blobs (kurumi_core/src/graph/serialize.rs; C ABI kurumi.h:407-453) ----

class InputRole(enum.IntEnum):
    """serialize.rs:28-33: a weight is bound by name from a weight table, a runtime input is fed."""
    Weight = 0
    Runtime = 1


class InputBinding(tuple):
    """(node, role, name) of one entry input (serialize.rs:35-41)."""
    __slots__ = ()

    def __new__(cls, node: int, role: InputRole, name: str):
        return super().__new__(cls, (int(node), InputRole(role), str(name)))

    node = property(lambda self: self[0])
    role = property(lambda self: self[1])
    name = property(lambda self: self[2])


class Entry:
    """One named entry point of a blob: its output node ids and input bindings."""

    def __init__(self, name: str, outputs: Sequence[int], inputs: Sequence[InputBinding]):
        self.name, self.outputs, self.inputs = name, list(outputs), list(inputs)

    def __repr__(self):
        return f"Entry({self.name!r}, outputs={self.outputs}, inputs={self.inputs})"


class Runnable:
    """A decoded blob: the rebuilt graph (ids preserved) and every entry (``MultiRunnable``).
    ``outputs``/``inputs`` are entry 0's, as in ``deserialize_graph``'s ``Runnable``."""

    def __init__(self, graph: Graph, entries: list[Entry]):
        self.graph, self.entries = graph, entries

    @property
    def outputs(self) -> list[int]:
        return self.entries[0].outputs

    @property
    def inputs(self) -> list[InputBinding]:
        return self.entries[0].inputs


def _bind_arrays(inputs: Sequence[InputBinding]):
    n = len(inputs)
    nodes = (C.c_uint32 * max(n, 1))(*[b[0] for b in inputs])
    roles = (C.c_uint8 * max(n, 1))(*[int(b[1]) for b in inputs])
    names = (C.c_char_p * max(n, 1))(*[str(b[2]).encode() for b in inputs])
    return nodes, roles, names


def _size_then_write(call) -> bytes:
    n = call(None, 0)
    if n == 0:  # a blob holds at least its magic, version and two counts: 0 is the error answer
        raise KuError(last_error())
    buf = C.create_string_buffer(max(n, 1))
    m = call(buf, n)
    if m != n:
        raise KuError(f"serialize: length changed {n} -> {m}")
    return buf.raw[:n]


def _serialize(cname: str, g: Graph, outputs: Sequence[int], inputs: Sequence[InputBinding]) -> bytes:
    outs = (C.c_uint32 * max(len(outputs), 1))(*outputs)
    nodes, roles, names = _bind_arrays(inputs)
    f = getattr(lib(), cname)
    return _size_then_write(lambda out, cap: f(g.h, outs, len(outputs), nodes, roles, names, len(inputs), out, cap))


def serialize_graph(g: Graph, outputs: Sequence[int], inputs: Sequence[InputBinding] = ()) -> bytes:
    """The whole arena in id order, one entry named "" (encode.rs:26-34)."""
    return _serialize("ku_graph_serialize", g, outputs, inputs)


def serialize_reachable(g: Graph, outputs: Sequence[int], inputs: Sequence[InputBinding] = ()) -> bytes:
    """Only the outputs' cone, dense-remapped; unreachable bindings dropped (encode.rs:42-44)."""
    return _serialize("ku_graph_serialize_reachable", g, outputs, inputs)


def serialize_multi(g: Graph, entries: Sequence[tuple[str, Sequence[int], Sequence[InputBinding]]]) -> bytes:
    """N named entries over one arena, pruned to the union of their cones (encode.rs:50-53)."""
    ne = len(entries)
    names = (C.c_char_p * max(ne, 1))(*[e[0].encode() for e in entries])
    oc = (C.c_uint32 * max(ne, 1))(*[len(e[1]) for e in entries])
    ic = (C.c_uint32 * max(ne, 1))(*[len(e[2]) for e in entries])
    flat_out = [o for e in entries for o in e[1]]
    outs = (C.c_uint32 * max(len(flat_out), 1))(*flat_out)
    nodes, roles, in_names = _bind_arrays([b for e in entries for b in e[2]])
    f = lib().ku_graph_serialize_multi
    return _size_then_write(lambda out, cap: f(g.h, ne, names, oc, outs, ic, nodes, roles, in_names, out, cap))


def _name(call) -> str:
    n = call(None, 0)
    buf = C.create_string_buffer(max(n, 1))
    call(buf, n)
    return buf.raw[:n].decode()


def deserialize_multi(blob: bytes) -> Runnable:
    """Rebuild a blob's graph and entries (decode.rs:28-31); raises KuError on a malformed blob."""
    L = lib()
    h = L.ku_graph_deserialize(bytes(blob), len(blob))
    if not h:
        raise KuError(last_error())
    try:
        entries = []
        for i in range(L.ku_runnable_entry_count(h)):
            name = _name(lambda out, cap: L.ku_runnable_entry_name(h, i, out, cap))
            outs = [L.ku_runnable_entry_output(h, i, j) for j in range(L.ku_runnable_entry_output_count(h, i))]
            ins = []
            for j in range(L.ku_runnable_entry_input_count(h, i)):
                nm = _name(lambda out, cap: L.ku_runnable_entry_input_name(h, i, j, out, cap))
                ins.append(InputBinding(L.ku_runnable_entry_input_node(h, i, j),
                                        L.ku_runnable_entry_input_role(h, i, j), nm))
            entries.append(Entry(name, outs, ins))
        graph = Graph(_handle=L.ku_runnable_take_graph(h))
    finally:
        L.ku_runnable_free(h)
    return Runnable(graph, entries)


def deserialize_graph(blob: bytes) -> Runnable:
    """Same as ``deserialize_multi``; ``outputs``/``inputs`` read entry 0 (decode.rs:20-24)."""
    return deserialize_multi(blob)


def quantize(w: np.ndarray, bits: int, group_size: int, symmetric: bool):
    """ku_quantize (kurumi_core/src/quant.rs:43-91): f32 [rows, cols] -> (packed u8 [rows, cols*bits/8],
    scales f16 bits u16 [rows, cols/group], mins u16 or None)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    if bits not in (2, 4, 8) or group_size <= 0 or cols % group_size or cols * bits % 8:
        raise KuError("quantize: bits must be 2, 4 or 8 and group_size must divide cols")
    packed = np.zeros((rows, cols * bits // 8), np.uint8)
    scales = np.zeros((rows, cols // group_size), np.uint16)
    mins = None if symmetric else np.zeros((rows, cols // group_size), np.uint16)
    lib().ku_quantize(w.ctypes.data_as(C.POINTER(C.c_float)), rows, cols, bits, group_size, int(symmetric),
                      packed.ctypes.data_as(C.c_char_p), scales.ctypes.data_as(C.POINTER(C.c_uint16)),
                      None if mins is None else mins.ctypes.data_as(C.POINTER(C.c_uint16)))
    return packed, scales, mins


def amp(g: Graph, root: int) -> int:
    """The reference's mixed-precision pass (graph/pass/amp.rs:16-40; kurumi.h:395 ku_amp)."""
    return g._n("ku_amp", root)


def amp_fp8(g: Graph, root: int) -> int:
    """The e4m3 mixed-precision pass (see include/kurumi_hip.h `ku_amp_fp8`)."""
    return g._n("ku_amp_fp8", root)


class HipPlan:
    """Device-resident plan: inputs uploaded once, launches stay on the GPU stream."""

    def __init__(self, backend: "HipBackend", g: Graph, roots: Sequence[int], feeds: dict[int, Tensor]):
        self._g = g
        self._b = backend
        arr = (C.c_uint32 * len(roots))(*roots)
        self._feeds = Feeds(feeds)
        self.h = lib().ku_hip_plan_new(g.h, arr, len(roots), backend.h, self._feeds.h)
        if not self.h:
            raise KuError(f"ku_hip_plan_new: {last_error()}")

    def feed(self, node: int, t: Tensor) -> None:
        """Upload a new value for one Input (same shape and dtype) into the plan's buffer."""
        th = t._handle()
        try:
            if lib().ku_hip_plan_feed(self.h, int(node), th) != 0:
                raise KuError(f"ku_hip_plan_feed: {last_error()}")
        finally:
            lib().ku_tensor_free(th)

    def launch(self, use_graph: bool = False) -> None:
        if lib().ku_hip_plan_launch(self.h, int(use_graph)) != 0:
            raise KuError(f"ku_hip_plan_launch: {last_error()}")

    def sync(self) -> None:
        if lib().ku_hip_plan_sync(self.h) != 0:
            raise KuError(f"ku_hip_plan_sync: {last_error()}")

    def output(self, i: int) -> Tensor:
        h = lib().ku_hip_plan_output(self.h, i)
        if not h:
            raise KuError(f"ku_hip_plan_output: {last_error()}")
        return Tensor._from_handle(h)

    def steps(self) -> list[str]:
        out = []
        for i in range(lib().ku_hip_plan_num_steps(self.h)):
            buf = C.create_string_buffer(512)
            lib().ku_hip_plan_step_label(self.h, i, buf, 512)
            out.append(buf.value.decode())
        return out

    def time_steps(self, iters: int) -> list[float]:
        n = lib().ku_hip_plan_num_steps(self.h)
        arr = (C.c_double * max(n, 1))()
        r = lib().ku_hip_plan_time_steps(self.h, iters, arr, n)
        if r < 0:
            raise KuError(f"ku_hip_plan_time_steps: {last_error()}")
        return list(arr[:n])

    def time(self, iters: int, use_graph: bool = False) -> float:
        ms = lib().ku_hip_plan_time(self.h, iters, int(use_graph))
        if ms < 0:
            raise KuError(f"ku_hip_plan_time: {last_error()}")
        return ms

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.ku_hip_plan_free(self.h)
            self.h = None


def time_plans(plans: Sequence[HipPlan], iters: int, use_graph: bool = False) -> float:
    """Average GPU ms of one round launching every plan once (ku_hip_plans_time)."""
    arr = (C.c_void_p * len(plans))(*[p.h for p in plans])
    ms = lib().ku_hip_plans_time(arr, len(plans), iters, int(use_graph))
    if ms < 0:
        raise KuError(f"ku_hip_plans_time: {last_error()}")
    return ms


class HipBackend:
    """`ku_backend_new(KU_HIP)`: the MI355X backend. Raises KuError when no device is usable."""

    KIND = 2

    def __init__(self):
        self.h = lib().ku_backend_new(self.KIND)
        if not self.h:
            raise KuError(f"ku_backend_new(KU_HIP): {last_error()}")

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.ku_backend_free(self.h)
            self.h = None

    name = "hip"

    def eval(self, g: Graph, node: int) -> Tensor:
        h = lib().ku_eval(g.h, node, self.h)
        if not h:
            raise KuError(f"ku_eval: {last_error()}")
        return Tensor._from_handle(h)

    def eval_with(self, g: Graph, node: int, feeds: dict[int, Tensor]) -> Tensor:
        f = Feeds(feeds)
        h = lib().ku_eval_with(g.h, node, self.h, f.h)
        if not h:
            raise KuError(f"ku_eval_with: {last_error()}")
        return Tensor._from_handle(h)

    def eval_many_with(self, g: Graph, ids: Sequence[int], feeds: dict[int, Tensor]) -> list[Tensor]:
        f = Feeds(feeds)
        arr = (C.c_uint32 * len(ids))(*ids)
        out = (C.c_void_p * len(ids))()
        if lib().ku_eval_many(g.h, arr, len(ids), self.h, f.h, out) != 0:
            raise KuError(f"ku_eval_many: {last_error()}")
        return [Tensor._from_handle(out[i]) for i in range(len(ids))]

    def plan(self, g: Graph, roots: Sequence[int], feeds: dict[int, Tensor]) -> HipPlan:
        return HipPlan(self, g, roots, feeds)

    def linear_e4m3(self, x: int, x_dtype: DType, wq: int, sw: int, y: int, y_dtype: DType, m: int, n: int, k: int,
                    stream: int | None = None) -> None:
        """ku_hip_linear_e4m3 on device pointers (ints): y = (e4m3(x / sx) @ wq^T) * sx * sw[n]."""
        if lib().ku_hip_linear_e4m3(self.h, x, int(x_dtype), wq, sw, y, int(y_dtype), m, n, k, stream) != 0:
            raise KuError(f"ku_hip_linear_e4m3: {last_error()}")

    def linear_e4m3_noalloc(self, x: int, x_dtype: DType, wq: int, sw: int, y: int, y_dtype: DType, m: int,
                            n: int, k: int, stream: int | None = None) -> None:
        """ku_hip_linear_e4m3_noalloc (static scratch, no allocation; m * k <= 16 MiB)."""
        linear_e4m3_noalloc(x, x_dtype, wq, sw, y, y_dtype, m, n, k, stream)

    def compile(self, g: Graph, node: int) -> "Plan":
        """kurumi.h:456 ku_plan_compile on this backend (ku_hip_plan_compile_on)."""
        return Plan(g, node, self)

    def profile(self) -> dict:
        keys = ["fused", "gemm", "attention", "upload", "download", "plans_built", "const_uploads", "const_entries"]
        arr = (C.c_uint64 * len(keys))()
        evals = lib().ku_hip_profile(self.h, arr, len(keys))
        return {"evals": evals, **dict(zip(keys, list(arr)))}


def linear_e4m3_noalloc(x: int, x_dtype: DType, wq: int, sw: int, y: int, y_dtype: DType, m: int, n: int, k: int,
                        stream: int | None = None) -> None:
    """ku_hip_linear_e4m3_noalloc on device pointers (current device; no backend needed)."""
    if lib().ku_hip_linear_e4m3_noalloc(x, int(x_dtype), wq, sw, y, int(y_dtype), m, n, k, stream) != 0:
        raise KuError(f"ku_hip_linear_e4m3_noalloc: {last_error()}")


class Plan:
    """Compile once, run per feeds (kurumi_core/src/realize/plan.rs:13-58; C ABI kurumi.h:455-458).
    Here a device plan replayed as one hipGraph launch per run. Without a backend it lives on the
    process-default KU_HIP backend (``ku_plan_compile``)."""

    def __init__(self, g: Graph, node: int, backend: "HipBackend | None" = None):
        self._b = backend
        if backend is None:
            self.h = lib().ku_plan_compile(g.h, node)
        else:
            self.h = lib().ku_hip_plan_compile_on(backend.h, g.h, node)
        if not self.h:
            raise KuError(f"ku_plan_compile: {last_error()}")

    def run(self, g: Graph, feeds: dict[int, Tensor]) -> Tensor:
        f = Feeds(feeds)
        h = lib().ku_plan_run(self.h, g.h, f.h)
        if not h:
            raise KuError(f"ku_plan_run: {last_error()}")
        return Tensor._from_handle(h)

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.ku_plan_free(self.h)
            self.h = None
