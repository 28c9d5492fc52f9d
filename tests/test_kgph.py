"""KGPH v2 graph blobs: encoder, decoder and their C ABI.

Mirrors the reference's codec tests (kurumi_core/src/graph/serialize/tests.rs:71-255): every op
round-trips, whole-arena / reachable / multi-entry blobs round-trip and compute the same values,
the committed 175-byte golden blob (tests/golden/graph_v2.kgph, the reference's own fixture
kurumi_core/tests/fixtures/graph_v2.kgph) is reproduced byte for byte from `golden_graph()` and
decodes to [12, 21], and malformed blobs are clean errors. Values are checked on the oracle here
and on the HIP backend in the `gpu` tests at the end.
"""
import ctypes as C
import random
import struct
from pathlib import Path

import numpy as np
import pytest

import kurumi_amd as K
from kurumi_amd import DType, Graph, InputBinding, InputRole, KuError, Tensor
from kutest import interpret

GOLDEN = Path(__file__).resolve().parent / "golden" / "graph_v2.kgph"
X6 = np.array([[1, 2, 3], [4, 5, 6]], np.float32)


def golden_graph():
    """serialize/tests.rs:191-199: an all-const graph, Sum{axis:1}(x + w)."""
    g = Graph()
    x = g.constant(X6)
    w = g.constant(np.full((2, 3), 2.0, np.float32))
    a = g.add(x, w)
    return g, [g.sum(a, 1)], []


def header(n_nodes: int) -> bytes:
    return b"KGPH\x02" + struct.pack("<I", n_nodes)


def entry_table(*entries) -> bytes:
    out = struct.pack("<I", len(entries))
    for name, outs in entries:
        out += struct.pack("<I", len(name)) + name + struct.pack("<I", len(outs))
        out += b"".join(struct.pack("<I", o) for o in outs) + struct.pack("<I", 0)
    return out


def const_f32(vals, shape) -> bytes:
    payload = np.asarray(vals, np.float32).tobytes()
    return (b"\x00" + bytes([DType.F32]) + struct.pack("<Q", len(payload)) + payload
            + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape) + struct.pack("<I", 0))


def rejects(blob: bytes, match: str | None = None):
    with pytest.raises(KuError, match=match):
        K.deserialize_graph(blob)


# ---------------- golden fixture ----------------

def test_golden_blob_is_stable():
    golden = GOLDEN.read_bytes()
    assert len(golden) == 175
    g, outs, ins = golden_graph()
    assert K.serialize_graph(g, outs, ins) == golden
    r = K.deserialize_graph(golden)
    assert r.outputs == [3] and r.inputs == []
    got = interpret(r.graph, r.outputs)[0].numpy()
    np.testing.assert_array_equal(got, np.array([12.0, 21.0], np.float32))


def test_golden_blob_layout_by_hand():
    """The fixture read field by field, independently of the decoder (serialize.rs:1-67)."""
    b = GOLDEN.read_bytes()
    assert b[:5] == b"KGPH\x02" and struct.unpack_from("<I", b, 5)[0] == 4
    p = 9
    for want in (X6.ravel(), np.full(6, 2.0, np.float32)):
        assert b[p] == 0 and b[p + 1] == DType.F32  # Const, F32 storage
        nb = struct.unpack_from("<Q", b, p + 2)[0]
        assert nb == 24
        np.testing.assert_array_equal(np.frombuffer(b, np.float32, 6, p + 10), want)
        p += 10 + nb
        assert struct.unpack_from("<IQQ", b, p) == (2, 2, 3)
        p += 20
        assert struct.unpack_from("<I", b, p)[0] == 0  # no sources
        p += 4
    assert b[p] == 7 and struct.unpack_from("<III", b, p + 1) == (2, 0, 1)  # Add(%0, %1)
    p += 13
    assert b[p] == 26 and struct.unpack_from("<QII", b, p + 1) == (1, 1, 2)  # Sum{axis:1}(%2)
    p += 17
    # one entry: name "", outputs [3], inputs []
    assert struct.unpack_from("<IIIII", b, p) == (1, 0, 1, 3, 0)
    assert p + 20 == len(b)


# ---------------- round trips ----------------

def test_graph_blob_round_trips():
    g = Graph()
    x = g.input([2, 3], DType.F32)
    w = g.constant(np.full((2, 3), 2.0, np.float32))
    a = g.add(x, w)
    m = g.mul(a, w)
    out = g.sum(m, 1)
    ins = [InputBinding(x, InputRole.Runtime, "x")]
    blob = K.serialize_graph(g, [out], ins)
    r = K.deserialize_graph(blob)
    assert r.outputs == [out] and r.inputs == ins
    feeds = {x: Tensor.from_numpy(X6)}
    want = interpret(g, [out], feeds)[0].numpy()
    got = interpret(r.graph, r.outputs, feeds)[0].numpy()
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(got, np.array([24.0, 42.0], np.float32))


def test_reachable_prunes_dead_nodes():
    g = Graph()
    x = g.input([2, 3], DType.F32)
    w = g.constant(np.full((2, 3), 2.0, np.float32))
    g.neg(w)  # dead
    a = g.add(x, w)
    out = g.sum(a, 1)
    ins = [InputBinding(x, InputRole.Runtime, "x")]
    full = K.serialize_graph(g, [out], ins)
    pruned = K.serialize_reachable(g, [out], ins)
    assert len(pruned) < len(full)
    r = K.deserialize_graph(pruned)
    assert len(r.inputs) == 1 and r.inputs[0].name == "x"
    got = interpret(r.graph, r.outputs, {r.inputs[0].node: Tensor.from_numpy(X6)})[0].numpy()
    np.testing.assert_array_equal(got, np.array([12.0, 21.0], np.float32))


def test_reachable_drops_unreachable_bindings_and_orders_post_dfs():
    g = Graph()
    x = g.input([3], DType.F32)
    y = g.input([3], DType.F32)  # bound but unused
    out = g.neg(x)
    blob = K.serialize_reachable(g, [out], [InputBinding(x, InputRole.Runtime, "x"),
                                            InputBinding(y, InputRole.Runtime, "y")])
    r = K.deserialize_graph(blob)
    assert r.inputs == [InputBinding(0, InputRole.Runtime, "x")] and r.outputs == [1]
    # post-order with the last source expanded first (inspect.rs:17-39): Add(a, b) emits b, a
    g = Graph()
    a = g.input([2], DType.F32)
    b = g.input([2], DType.F32)
    s = g.add(a, b)
    r = K.deserialize_graph(K.serialize_reachable(g, [s], [InputBinding(a, InputRole.Runtime, "a"),
                                                           InputBinding(b, InputRole.Weight, "b")]))
    assert r.inputs == [InputBinding(1, InputRole.Runtime, "a"), InputBinding(0, InputRole.Weight, "b")]


def test_multi_entry_round_trips():
    g = Graph()
    x = g.input([2, 3], DType.F32)
    w = g.constant(np.full((2, 3), 2.0, np.float32))
    a = g.add(x, w)
    fwd = g.sum(a, 1)
    bwd = g.sum(g.mul(a, w), 1)
    fwd_in = [InputBinding(x, InputRole.Runtime, "x")]
    bwd_in = [InputBinding(x, InputRole.Runtime, "x"), InputBinding(a, InputRole.Weight, "a")]
    blob = K.serialize_multi(g, [("forward", [fwd], fwd_in), ("forward_backward", [bwd], bwd_in)])
    mr = K.deserialize_multi(blob)
    assert [e.name for e in mr.entries] == ["forward", "forward_backward"]
    assert len(mr.entries[0].inputs) == 1 and len(mr.entries[1].inputs) == 2
    assert mr.entries[1].inputs[1].name == "a" and mr.entries[1].inputs[1].role == InputRole.Weight
    xn = mr.entries[0].inputs[0].node
    assert mr.entries[1].inputs[0].node == xn
    f, b = interpret(mr.graph, [mr.entries[0].outputs[0], mr.entries[1].outputs[0]], {xn: Tensor.from_numpy(X6)})
    np.testing.assert_array_equal(f.numpy(), [12.0, 21.0])
    np.testing.assert_array_equal(b.numpy(), [24.0, 42.0])
    r = K.deserialize_graph(blob)
    assert r.outputs == mr.entries[0].outputs and r.inputs == mr.entries[0].inputs


def every_op_graph():
    """A graph holding each of the 41 op kinds of this IR at least once."""
    g = Graph()
    x = g.input([2, 4], DType.F32)
    xi = g.input([2, 4], DType.I32)
    c = g.constant(np.arange(8, dtype=np.float32).reshape(2, 4))
    io = g.iota([2, 4], 1, DType.I32)
    ru = g.rand_uniform([2, 4], 7)  # Const seed + RandUniform
    outs = [ru]
    outs.append(g.cast(xi, DType.F32))
    outs.append(g.bitcast(xi, DType.U32))
    outs.append(g.detach(x))
    outs += [g.add(x, c), g.mul(x, c), g.max(x, c), g.neg(x)]
    outs += [g.idiv(xi, io), g.bit_and(xi, io), g.bit_or(xi, io), g.bit_xor(xi, io), g.shl(xi, io), g.shr(xi, io)]
    lt = g.lt(x, c)
    outs += [lt, g.eq(x, c), g.where(lt, x, c)]
    outs += [g.recip(x), g.sqrt(x), g.exp2(x), g.log2(x), g.sin(x), g.floor(x)]
    outs += [g.sum(x, 1), g.prod(x, 0), g.reduce_max(x, 1), g.argmax(x, 1), g.argmin(x, 0)]
    outs += [g.softmax(x, 1), g.rmsnorm(x, 1, 1e-6)]
    q = g.input([1, 2, 8, 4], DType.F32)
    outs.append(g.sdpa_fused(q, q, q, True))
    outs += [g.reshape(x, [4, 2]), g.permute(x, [1, 0]), g.expand(g.reshape(x, [2, 1, 4]), [2, 3, 4])]
    outs += [g.slice_step(x, [(0, 2, 1), (1, 4, 2)]), g.flip(x, [0, 1]), g.pad(x, [(1, 0), (0, 2)])]
    outs.append(g.dot_general(x, c, [1], [1], [0], [0]))
    packed, scales, mins = K.quantize(np.arange(32, dtype=np.float32).reshape(4, 8), 4, 8, False)
    qw = g.constant_bytes(DType.U8, packed.tobytes(), packed.shape)
    sc = g.constant_bytes(DType.F16, scales.tobytes(), scales.shape)
    mn = g.constant_bytes(DType.F16, mins.tobytes(), mins.shape)
    xq = g.reshape(x, [1, 8])
    outs += [g.quant_matmul(xq, qw, sc, mn, 4, 8), g.quant_matmul(xq, qw, sc, None, 4, 8)]
    return g, outs


def test_every_op_round_trips():
    g, outs = every_op_graph()
    blob = K.serialize_graph(g, outs)
    r = K.deserialize_graph(blob)
    assert K.serialize_graph(r.graph, r.outputs) == blob  # encode(decode(b)) == b
    kinds = set(blob_op_tags(blob))
    assert kinds == set(range(41)), sorted(set(range(41)) - kinds)
    for o in outs:
        assert r.graph.shape(o) == g.shape(o) and r.graph.dtype(o) == g.dtype(o)


def blob_op_tags(blob: bytes) -> list[int]:
    """Op tag of every node record, walking the blob with the layouts of encode/op.rs."""
    p, tags = 9, []
    for _ in range(struct.unpack_from("<I", blob, 5)[0]):
        tags.append(blob[p])
        p = node_end(blob, p)
    return tags


def node_end(b: bytes, p: int) -> int:
    """Offset after the node record starting at p (the attribute layouts of encode/op.rs)."""
    tag = b[p]
    p += 1

    def vec(p):
        n = struct.unpack_from("<I", b, p)[0]
        return p + 4 + 8 * n

    if tag == 0:
        nb = struct.unpack_from("<Q", b, p + 1)[0]
        p = vec(p + 9 + nb)
    elif tag == 1:
        p = vec(p) + 1
    elif tag == 2:
        p = vec(p) + 9
    elif tag == 3:
        p = vec(p)
    elif tag in (4, 5):
        p += 1
    elif tag in (26, 27, 28, 30):
        p += 8
    elif tag == 29:
        p += 9
    elif tag == 31:
        p += 12
    elif tag == 32:
        p += 1
    elif tag in (33, 34, 35, 37):
        p = vec(p)
    elif tag == 36:
        p += 4 + 24 * struct.unpack_from("<I", b, p)[0]
    elif tag == 38:
        p += 4 + 16 * struct.unpack_from("<I", b, p)[0]
    elif tag == 39:
        for _ in range(4):
            p = vec(p)
    elif tag == 40:
        p += 10
    ns = struct.unpack_from("<I", b, p)[0]
    return p + 4 + 4 * ns


def test_const_payload_follows_from_bytes():
    """decode/op.rs:13-23 + convert.rs:105-124: a trailing partial element is dropped, bool bytes
    normalise to 0/1."""
    vals = np.array([1.5, -2.0], np.float32).tobytes() + b"\x07"  # 9 bytes: two f32 + a stray byte
    node = b"\x00" + bytes([DType.F32]) + struct.pack("<Q", 9) + vals + struct.pack("<IQ", 1, 2) + struct.pack("<I", 0)
    r = K.deserialize_graph(header(1) + node + entry_table((b"", [0])))
    np.testing.assert_array_equal(interpret(r.graph, [0])[0].numpy(), [1.5, -2.0])
    node = b"\x00" + bytes([DType.BOOL]) + struct.pack("<Q", 3) + b"\x00\x05\x01" + struct.pack("<IQ", 1, 3)
    r = K.deserialize_graph(header(1) + node + struct.pack("<I", 0) + entry_table((b"", [0])))
    assert interpret(r.graph, [0])[0].numpy().view(np.uint8).tolist() == [0, 1, 1]


def test_rand_uniform_replays_with_its_seed():
    g = Graph()
    u = g.rand_uniform([16], 1234)
    r = K.deserialize_graph(K.serialize_graph(g, [u]))
    np.testing.assert_array_equal(interpret(r.graph, r.outputs)[0].numpy(), interpret(g, [u])[0].numpy())


# ---------------- rejections (serialize/tests.rs:223-255 and this decoder's own guards) ----------------

def test_rejects_bad_magic_and_version():
    rejects(b"XXXX\x01", "bad magic")
    rejects(b"", "bad magic")
    rejects(b"KGPH\x01" + struct.pack("<I", 0), "unsupported graph blob version 1")


def test_rejects_forward_src_ref():
    rejects(header(1) + b"\x07" + struct.pack("<II", 1, 0), r"node 0 references source 0 \(not yet built\)")


def test_rejects_const_payload_underfill():
    node = b"\x00" + bytes([DType.F32]) + struct.pack("<Q", 4) + struct.pack("<f", 1.0) + struct.pack("<IQ", 1, 2)
    rejects(header(1) + node, "Const payload has 1 elements")


def test_rejects_every_truncation_of_the_golden_blob():
    golden = GOLDEN.read_bytes()
    for n in range(len(golden)):
        rejects(golden[:n])


def test_rejects_entryless_blob_and_bad_fields():
    rejects(header(1) + const_f32([1.0], [1]) + struct.pack("<I", 0), "no entries")
    rejects(header(1) + b"\x00\x63", "unknown dtype tag 99")
    rejects(header(1) + b"\x63", "unknown op tag 99")
    rejects(header(1) + b"\x29", r"Solve \(tag 41\)")
    body = header(1) + const_f32([1.0, 2.0], [2])
    rejects(body + struct.pack("<I", 1) + struct.pack("<IIII", 0, 1, 0, 1) + struct.pack("<IBI", 0, 2, 0),
            "bad input role 2")
    rejects(body + struct.pack("<II", 1, 2) + b"\xc3\x28" + struct.pack("<II", 0, 0), "invalid utf8")
    rejects(body + struct.pack("<II", 1, 2) + b"\xe0\x80" + struct.pack("<II", 0, 0), "invalid utf8")
    sum_node = b"\x1d" + struct.pack("<Q", 0) + b"\x02" + struct.pack("<II", 1, 0)
    rejects(body[:5] + struct.pack("<I", 2) + body[9:] + sum_node, "unknown argkind 2")


def test_rejects_what_the_builders_reject():
    c = const_f32([1.0, 2.0, 3.0, 4.0], [4])
    rejects(header(2) + c + b"\x07" + struct.pack("<II", 1, 0), "Add takes 2 sources, got 1")
    reshape = b"\x21" + struct.pack("<IQ", 1, 3) + struct.pack("<II", 1, 0)
    rejects(header(2) + c + reshape, "reshape: numel")
    sum_ax = b"\x1a" + struct.pack("<Q", 5) + struct.pack("<II", 1, 0)
    rejects(header(2) + c + sum_ax, "axis 5 out of range")
    big = b"\x01" + struct.pack("<IQQ", 2, 1 << 40, 1 << 40) + bytes([DType.F32]) + struct.pack("<I", 0)
    rejects(header(1) + big, "overflows")
    # a shape that fits but whose outer product does not
    inp = b"\x01" + struct.pack("<IQ", 1, 1 << 40) + bytes([DType.F32]) + struct.pack("<I", 0)
    dot = b"\x27" + struct.pack("<IIII", 0, 0, 0, 0) + struct.pack("<III", 2, 0, 0)
    rejects(header(2) + inp + dot, "overflows")


def test_mutated_blobs_decode_or_fail_cleanly():
    """Byte flips of real blobs: every result is a graph or a KuError, never a crash."""
    g, outs = every_op_graph()
    blobs = [GOLDEN.read_bytes(), K.serialize_graph(g, outs)]
    rng = random.Random(20261201)
    ok = bad = 0
    for i in range(3000):
        b = bytearray(blobs[i % 2])
        for _ in range(rng.randint(1, 4)):
            b[rng.randrange(len(b))] = rng.randrange(256)
        try:
            K.deserialize_graph(bytes(b))
            ok += 1
        except KuError:
            bad += 1
    assert ok + bad == 3000 and bad > 0


# ---------------- C ABI semantics ----------------

def test_runnable_accessors_and_take_graph():
    L = K.lib()
    golden = GOLDEN.read_bytes()
    h = L.ku_graph_deserialize(golden, len(golden))
    assert h
    try:
        assert L.ku_runnable_entry_count(h) == 1 and L.ku_runnable_output_count(h) == 1
        assert L.ku_runnable_output(h, 0) == 3 and L.ku_runnable_output(h, 1) == K.KU_ERR
        assert L.ku_runnable_input_count(h) == 0 and L.ku_runnable_input_node(h, 0) == K.KU_ERR
        assert L.ku_runnable_input_role(h, 0) == K.KU_ERR and L.ku_runnable_input_name(h, 0, None, 0) == 0
        assert L.ku_runnable_entry_name(h, 0, None, 0) == 0 and L.ku_runnable_entry_output_count(h, 5) == 0
        g1 = L.ku_runnable_take_graph(h)
        g2 = L.ku_runnable_take_graph(h)  # the second take gets an empty graph
        assert L.ku_node_rank(g1, 3) == 1 and L.ku_node_rank(g2, 0) == C.c_size_t(-1).value
        L.ku_graph_free(g1)
        L.ku_graph_free(g2)
    finally:
        L.ku_runnable_free(h)
    assert L.ku_runnable_entry_count(None) == 0 and L.ku_runnable_output(None, 0) == K.KU_ERR
    assert not L.ku_runnable_take_graph(None)
    assert L.ku_graph_serialize(None, None, 0, None, None, None, 0, None, 0) == 0
    assert "null graph" in K.last_error()
    assert not L.ku_graph_deserialize(None, 0)


def test_size_then_write_and_lossy_names():
    L = K.lib()
    g = Graph()
    x = g.input([2], DType.F32)
    y = g.neg(x)
    outs = (C.c_uint32 * 1)(y)
    nodes = (C.c_uint32 * 1)(x)
    roles = (C.c_uint8 * 1)(0)
    names = (C.c_char_p * 1)(b"w\xff\xe2\x82x")  # invalid bytes become U+FFFD, one per maximal prefix
    n = L.ku_graph_serialize(g.h, outs, 1, nodes, roles, names, 1, None, 0)
    part = C.create_string_buffer(8)
    assert L.ku_graph_serialize(g.h, outs, 1, nodes, roles, names, 1, part, 8) == n
    full = C.create_string_buffer(n)
    L.ku_graph_serialize(g.h, outs, 1, nodes, roles, names, 1, full, n)
    assert part.raw == full.raw[:8]
    r = K.deserialize_graph(full.raw)
    assert r.inputs == [InputBinding(x, InputRole.Weight, "w\ufffd\ufffdx")]
    with pytest.raises(KuError, match="out of range"):
        K.serialize_reachable(g, [99])


# ---------------- device: decoded graphs run on the HIP backend ----------------

@pytest.mark.gpu
def test_golden_blob_evaluates_on_device(hip):
    print("kgph golden on device", flush=True)
    r = K.deserialize_graph(GOLDEN.read_bytes())
    np.testing.assert_array_equal(hip.eval(r.graph, r.outputs[0]).numpy(), [12.0, 21.0])


@pytest.mark.gpu
def test_decoded_hot_path_graph_matches_the_live_one(hip):
    """A cfg-2 shaped graph (softmax + argmax) sent through a blob gives bit-identical results."""
    print("kgph softmax+argmax round trip", flush=True)
    g = Graph()
    x = g.input([64, 1000], DType.F32)
    y = g.softmax(x, 1)
    a = g.cast(g.argmax(y, 1), DType.I32)
    blob = K.serialize_reachable(g, [y, a], [InputBinding(x, InputRole.Runtime, "logits")])
    r = K.deserialize_graph(blob)
    xv = np.random.default_rng(5).standard_normal((64, 1000)).astype(np.float32)
    live = hip.eval_many_with(g, [y, a], {x: Tensor.from_numpy(xv)})
    dec = hip.eval_many_with(r.graph, r.outputs, {r.inputs[0].node: Tensor.from_numpy(xv)})
    for p, q in zip(live, dec):
        np.testing.assert_array_equal(p.numpy(), q.numpy())
