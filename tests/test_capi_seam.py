"""The collision-free entry set (ku_hip_api) on the CPU, no GPU calls.

kurumi's own library exports the same unprefixed ku_* names as libkurumi_hip.so
(kurumi/Cargo.toml:12-13, kurumi/src/capi/eval.rs:10-23). A stand-in library exporting those
names is loaded globally first, so every lookup of a ku_* name by the dynamic linker finds the
stand-in; calls through the table that ku_hip_api returns, including the library's own internal
calls between entry points, must still reach libkurumi_hip.so and never the stand-in.
"""
import ctypes as C
import json
import subprocess
import sys
import textwrap
from pathlib import Path

import numpy as np
import pytest

import kurumi_amd as K
from kurumi_amd import DType, Graph

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "kurumi_amd" / "libkurumi_hip.so"

# Every stand-in function counts its calls and returns a sentinel no real call returns.
STANDIN = r"""
#include <stddef.h>
#include <stdint.h>
static int calls = 0;
int standin_calls(void) { return calls; }
const char *ku_last_error(void) { calls++; return "stand-in"; }
void *ku_backend_new(uint32_t k) { calls++; return (void *)0x5152; }
void ku_backend_free(void *b) { calls++; }
void *ku_graph_new(void) { calls++; return (void *)0x5151; }
void ku_graph_free(void *g) { calls++; }
void *ku_graph_deserialize(const uint8_t *b, size_t n) { calls++; return (void *)0x5153; }
void *ku_runnable_take_graph(void *h) { calls++; return (void *)0x5154; }
size_t ku_runnable_output_count(const void *h) { calls++; return 77; }
uint32_t ku_runnable_output(const void *h, size_t i) { calls++; return 77; }
size_t ku_runnable_input_count(const void *h) { calls++; return 77; }
uint32_t ku_runnable_input_node(const void *h, size_t i) { calls++; return 77; }
size_t ku_runnable_input_name(const void *h, size_t i, uint8_t *o, size_t c) { calls++; return 77; }
size_t ku_runnable_entry_output_count(const void *h, size_t i) { calls++; return 77; }
uint32_t ku_runnable_entry_output(const void *h, size_t i, size_t j) { calls++; return 77; }
size_t ku_runnable_entry_input_count(const void *h, size_t i) { calls++; return 77; }
uint32_t ku_runnable_entry_input_node(const void *h, size_t i, size_t j) { calls++; return 77; }
size_t ku_runnable_entry_input_name(const void *h, size_t i, size_t j, uint8_t *o, size_t c) { calls++; return 77; }
void ku_runnable_free(void *h) { calls++; }
void *ku_feeds_new(void) { calls++; return (void *)0x5155; }
void ku_feeds_free(void *f) { calls++; }
void ku_feeds_set(void *f, uint32_t n, const void *t) { calls++; }
void *ku_tensor_new(uint32_t d, const uint8_t *p, size_t n, const size_t *s, size_t r) { calls++; return (void *)0x5156; }
void ku_tensor_free(void *t) { calls++; }
size_t ku_tensor_rank(const void *t) { calls++; return 77; }
void ku_tensor_shape(const void *t, size_t *o) { calls++; }
uint32_t ku_tensor_dtype(const void *t) { calls++; return 77; }
size_t ku_tensor_nbytes(const void *t) { calls++; return 77; }
void ku_tensor_bytes(const void *t, uint8_t *o) { calls++; }
size_t ku_node_count(const void *g, uint32_t r) { calls++; return 77; }
size_t ku_dump(const void *g, uint32_t r, uint8_t *o, size_t c) { calls++; return 77; }
void *ku_eval(void *g, uint32_t n, const void *b) { calls++; return (void *)0x5157; }
void *ku_eval_with(void *g, uint32_t n, const void *b, const void *f) { calls++; return (void *)0x5158; }
int32_t ku_eval_many(void *g, const uint32_t *ids, size_t n, const void *b, const void *f, void **out) { calls++; return 0; }
void *ku_hip_plan_compile_on(const void *b, const void *g, uint32_t n) { calls++; return (void *)0x5159; }
void *ku_plan_run(const void *p, const void *g, const void *f) { calls++; return (void *)0x515a; }
void ku_plan_free(void *p) { calls++; }
"""

# Field order of KuHipApi in include/kurumi_hip.h (after version and size).
FIELDS = ["last_error", "backend_new", "backend_free", "graph_new", "graph_free", "graph_deserialize",
          "runnable_take_graph", "runnable_output_count", "runnable_output", "runnable_input_count",
          "runnable_input_node", "runnable_input_name", "runnable_free", "eval", "eval_with", "eval_many",
          "plan_compile_on", "plan_run", "plan_free", "feeds_new", "feeds_free", "feeds_set", "tensor_new",
          "tensor_free", "tensor_rank", "tensor_shape", "tensor_dtype", "tensor_nbytes", "tensor_bytes",
          "node_count", "dump"]

CHILD = textwrap.dedent(r"""
    import ctypes as C, json, sys
    standin_path, lib_path, blob_path = sys.argv[1:4]
    S = C.CDLL(standin_path, mode=C.RTLD_GLOBAL)   # first in the global scope
    L = C.CDLL(lib_path, mode=C.RTLD_GLOBAL)
    FIELDS, F32 = json.loads(sys.argv[4]), int(sys.argv[5])
    P, Z, U32 = C.c_void_p, C.c_size_t, C.c_uint32
    class Api(C.Structure):
        _fields_ = [("version", U32), ("size", U32)] + [(f, P) for f in FIELDS]
    L.ku_hip_api.restype = C.POINTER(Api)
    L.ku_hip_api.argtypes = [U32]
    out = {}
    out["bad_version_null"] = not bool(L.ku_hip_api(99))
    T = L.ku_hip_api(1).contents
    out["version"], out["size"] = T.version, T.size
    fn = lambda name, res, *args: C.CFUNCTYPE(res, *args)(getattr(T, name))
    # backend: libkurumi_hip's own refusal of KU_CPU and its own error text
    out["cpu_backend_null"] = fn("backend_new", P, U32)(0) is None
    out["error"] = fn("last_error", C.c_char_p)().decode()
    # KGPH decode; runnable_output / input_* call the entry_* functions inside the library
    blob = open(blob_path, "rb").read()
    r = fn("graph_deserialize", P, C.c_char_p, Z)(blob, len(blob))
    out["outputs"] = [fn("runnable_output", U32, P, Z)(r, i) for i in range(fn("runnable_output_count", Z, P)(r))]
    out["inputs"] = [fn("runnable_input_node", U32, P, Z)(r, i) for i in range(fn("runnable_input_count", Z, P)(r))]
    buf = C.create_string_buffer(64)
    n = fn("runnable_input_name", Z, P, Z, C.c_char_p, Z)(r, 0, buf, 64)
    out["input_name"] = buf.raw[:n].decode()
    g = fn("runnable_take_graph", P, P)(r)
    fn("runnable_free", None, P)(r)
    n = fn("dump", Z, P, U32, C.c_char_p, Z)(g, out["outputs"][0], None, 0)
    buf = C.create_string_buffer(n)
    fn("dump", Z, P, U32, C.c_char_p, Z)(g, out["outputs"][0], buf, n)
    out["dump"] = buf.raw[:n].decode()
    out["node_count"] = fn("node_count", Z, P, U32)(g, out["outputs"][0])
    fn("graph_free", None, P)(g)
    # tensors and feeds
    data = (C.c_float * 4)(1.5, -2.0, 3.25, 8.0)
    shape = (Z * 2)(2, 2)
    t = fn("tensor_new", P, U32, P, Z, P, Z)(F32, C.addressof(data), 16, C.addressof(shape), 2)
    out["tensor_dtype"] = fn("tensor_dtype", U32, P)(t)
    out["tensor_rank"] = fn("tensor_rank", Z, P)(t)
    out["tensor_nbytes"] = fn("tensor_nbytes", Z, P)(t)
    back = (C.c_float * 4)()
    fn("tensor_bytes", None, P, P)(t, C.addressof(back))
    out["tensor"] = list(back)
    f = fn("feeds_new", P)()
    fn("feeds_set", None, P, U32, P)(f, 0, t)
    fn("feeds_free", None, P)(f)
    fn("tensor_free", None, P)(t)
    gg = fn("graph_new", P)()
    out["graph_new_real"] = gg not in (None, 0x5151)
    fn("graph_free", None, P)(gg)
    S.standin_calls.restype = C.c_int
    out["standin_calls_through_table"] = S.standin_calls()
    # the hazard is real: a lookup of the plain name by the dynamic linker finds the stand-in
    glob = C.CDLL(None)
    glob.ku_graph_new.restype = P
    out["global_graph_new"] = glob.ku_graph_new()
    out["standin_calls_after_plain_name"] = S.standin_calls()
    print(json.dumps(out))
""")


def test_table_reaches_this_library_when_same_names_are_loaded_first(tmp_path):
    src = tmp_path / "standin.c"
    src.write_text(STANDIN)
    standin = tmp_path / "libstandin.so"
    subprocess.run(["gcc", "-shared", "-fPIC", "-O1", "-o", str(standin), str(src)], check=True)
    # a blob with one named runtime input: y = x * x + 1
    g = Graph()
    x = g.input([2, 2], DType.F32)
    y = g.add(g.mul(x, x), g.scalar(x, 1.0))
    blob = tmp_path / "g.kgph"
    blob.write_bytes(K.serialize_graph(g, [y], [K.InputBinding(x, K.InputRole.Runtime, "x")]))
    want = K.deserialize_graph(blob.read_bytes())
    r = subprocess.run([sys.executable, "-c", CHILD, str(standin), str(LIB), str(blob), json.dumps(FIELDS),
                        str(int(DType.F32))],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["bad_version_null"]
    assert out["version"] == 1
    assert out["size"] == 8 + 8 * len(FIELDS)
    assert out["cpu_backend_null"] and "libkurumi_hip provides KU_HIP" in out["error"]
    assert out["outputs"] == want.outputs and out["inputs"] == [b.node for b in want.inputs]
    assert out["input_name"] == "x" == want.inputs[0].name
    assert out["dump"] == want.graph.dump(want.outputs[0])
    assert out["node_count"] == want.graph.node_count(want.outputs[0])
    assert out["tensor_rank"] == 2 and out["tensor_nbytes"] == 16 and out["tensor_dtype"] == int(DType.F32)
    np.testing.assert_array_equal(out["tensor"], [1.5, -2.0, 3.25, 8.0])
    assert out["graph_new_real"]
    assert out["standin_calls_through_table"] == 0
    assert out["global_graph_new"] == 0x5151 and out["standin_calls_after_plain_name"] == 1


def test_table_matches_the_exported_definitions():
    # in a process without the stand-in, each table entry is the exported function itself
    L = K.lib()
    L.ku_hip_api.restype = C.c_void_p
    L.ku_hip_api.argtypes = [C.c_uint32]
    base = L.ku_hip_api(1)
    assert base
    ptrs = (C.c_void_p * len(FIELDS)).from_address(base + 8)
    for i, f in enumerate(FIELDS):
        name = {"plan_compile_on": "ku_hip_plan_compile_on"}.get(f, "ku_" + f)
        assert ptrs[i] == C.cast(getattr(L, name), C.c_void_p).value, f


# The backend seam on the device: a KGPH blob evaluated on KU_HIP, and planned and replayed,
# entirely through the table, with the same-named stand-in loaded first.
GPU_CHILD = textwrap.dedent(r"""
    import ctypes as C, json, sys
    import numpy as np
    standin_path, lib_path, blob_path, x_path = sys.argv[1:5]
    S = C.CDLL(standin_path, mode=C.RTLD_GLOBAL)
    L = C.CDLL(lib_path, mode=C.RTLD_GLOBAL)
    FIELDS, F32 = json.loads(sys.argv[5]), int(sys.argv[6])
    P, Z, U32 = C.c_void_p, C.c_size_t, C.c_uint32
    class Api(C.Structure):
        _fields_ = [("version", U32), ("size", U32)] + [(f, P) for f in FIELDS]
    L.ku_hip_api.restype = C.POINTER(Api)
    T = L.ku_hip_api(1).contents
    fn = lambda name, res, *args: C.CFUNCTYPE(res, *args)(getattr(T, name))
    b = fn("backend_new", P, U32)(2)
    assert b, fn("last_error", C.c_char_p)()
    blob = open(blob_path, "rb").read()
    r = fn("graph_deserialize", P, C.c_char_p, Z)(blob, len(blob))
    outs = [fn("runnable_output", U32, P, Z)(r, i) for i in range(fn("runnable_output_count", Z, P)(r))]
    xin = fn("runnable_input_node", U32, P, Z)(r, 0)
    g = fn("runnable_take_graph", P, P)(r)
    fn("runnable_free", None, P)(r)
    x = np.load(x_path)
    shape = (Z * 2)(*x.shape)
    t = fn("tensor_new", P, U32, P, Z, P, Z)(F32, x.ctypes.data, x.nbytes, C.addressof(shape), 2)
    f = fn("feeds_new", P)()
    fn("feeds_set", None, P, U32, P)(f, xin, t)
    ids = (U32 * len(outs))(*outs)
    res = (P * len(outs))()
    assert fn("eval_many", C.c_int32, P, P, Z, P, P, P)(g, ids, len(outs), b, f, res) == 0, fn("last_error", C.c_char_p)()
    def fetch(h):
        n = fn("tensor_nbytes", Z, P)(h)
        buf = (C.c_uint8 * n)()
        fn("tensor_bytes", None, P, P)(h, buf)
        fn("tensor_free", None, P)(h)
        return bytes(buf).hex()
    got = [fetch(res[i]) for i in range(len(outs))]
    p = fn("plan_compile_on", P, P, P, U32)(b, g, outs[0])
    assert p, fn("last_error", C.c_char_p)()
    replay = fetch(fn("plan_run", P, P, P, P)(p, g, f))
    fn("plan_free", None, P)(p)
    fn("feeds_free", None, P)(f)
    fn("tensor_free", None, P)(t)
    fn("graph_free", None, P)(g)
    fn("backend_free", None, P)(b)
    S.standin_calls.restype = C.c_int
    print(json.dumps({"got": got, "replay": replay, "standin_calls": S.standin_calls()}))
""")


@pytest.mark.gpu
def test_table_evaluates_and_replays_on_the_gpu_with_same_names_loaded_first(hip, tmp_path):
    src = tmp_path / "standin.c"
    src.write_text(STANDIN)
    standin = tmp_path / "libstandin.so"
    subprocess.run(["gcc", "-shared", "-fPIC", "-O1", "-o", str(standin), str(src)], check=True)
    g = Graph()
    x = g.input([64, 1000], DType.F32)
    y = g.softmax(x, 1)
    a = g.cast(g.argmax(y, 1), DType.I32)
    blob = tmp_path / "g.kgph"
    blob.write_bytes(K.serialize_graph(g, [y, a], [K.InputBinding(x, K.InputRole.Runtime, "x")]))
    xv = np.random.default_rng(4).standard_normal((64, 1000)).astype(np.float32) * 3
    np.save(tmp_path / "x.npy", xv)
    # the same graph through the plain names, in this process (no stand-in here)
    want = hip.eval_many_with(g, [y, a], {x: K.Tensor.from_numpy(xv)})
    r = subprocess.run([sys.executable, "-c", GPU_CHILD, str(standin), str(LIB), str(blob), str(tmp_path / "x.npy"),
                        json.dumps(FIELDS), str(int(DType.F32))], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-3000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["standin_calls"] == 0
    assert bytes.fromhex(out["got"][0]) == want[0].numpy().tobytes()
    assert bytes.fromhex(out["got"][1]) == want[1].numpy().tobytes()
    assert bytes.fromhex(out["replay"]) == want[0].numpy().tobytes()
