"""Seeded random graphs for the device-vs-oracle differential fuzz.

Each graph starts from three constants (two matrices, one tensor of random rank) and grows by
random steps drawn from the IR this backend runs: elementwise unary and binary ops, casts
between float dtypes, movement (permute, reshape, slice with steps, flip, pad, broadcast),
reductions (sum, max, softmax, and argmax of a constant), contractions and attention. The last
node and two random earlier ones are the roots, so one plan stores several outputs. Float graphs
draw values in [-4, 4]; integer graphs draw in [0, 8) so every op stays exact and in range in
every integer dtype (the same spirit as kurumi_metal/src/tests/fuzz.rs:183-225, generated
independently here).

Contractions come in two kinds: small ones between matrices of the graph (f32 only), and ones
with a contraction length that is a multiple of 64, in every float dtype, so that the 16-bit
dtypes take the MFMA GEMM (plain, NT, batched, transposed lhs). Their operands are multiples of
1/16 in [-1, 1]: every product and partial sum is then exact in f32 whatever the summation
order, so the device and the oracle agree bit for bit on the contraction and it may feed any
later op; every such contraction is also a root, so none is left unevaluated. Attention (fused or decomposed, causal or not, head sizes 32 / 64 / 128) takes q, k, v
of the same kind; its result is not exact (exponentials), so it only ever becomes a root, and
`attn_roots` lists those roots for a norm-wise bar.
"""
from __future__ import annotations

import numpy as np

from kurumi_amd import DType, Graph

FLOATS = (DType.F32, DType.BF16, DType.F16)
INTS = (DType.I32, DType.I64, DType.U32, DType.U8)


def _const(g: Graph, rng, shape, dt: DType):
    n = int(np.prod(shape))
    if dt in INTS:
        vals = rng.integers(0, 8, n).astype(dt.storage)
        return g.constant_bytes(dt, vals.tobytes(), shape)
    vals = (rng.integers(-400, 401, n) / 100.0).astype(np.float32)
    node = g.constant_bytes(DType.F32, vals.tobytes(), shape)
    return node if dt == DType.F32 else g.cast(node, dt)


def _factor(rng, n):
    if n <= 1 or rng.integers(2) == 0:
        return [n]
    divs = [d for d in range(1, n + 1) if n % d == 0]
    d = int(divs[rng.integers(len(divs))])
    return [d, n // d]


def _movement(rng, g: Graph, node, shape):
    k = int(rng.integers(6))
    r = len(shape)
    if k == 0:
        p = list(rng.permutation(r))
        return g.permute(node, p), [shape[i] for i in p]
    if k == 1:
        ns = _factor(rng, int(np.prod(shape)))
        return g.reshape(node, ns), ns
    if k == 2:
        rg = []
        for d in shape:
            a = int(rng.integers(d))
            b = a + 1 + int(rng.integers(d - a))
            st = 1 + int(rng.integers(2))
            rg.append((a, b, st))
        return g.slice_step(node, rg), [(b - a + st - 1) // st for a, b, st in rg]
    if k == 3:
        axes = [i for i in range(r) if rng.integers(2)]
        return g.flip(node, axes), list(shape)
    if k == 4:
        pads = [(int(rng.integers(3)), int(rng.integers(3))) for _ in shape]
        return g.pad(node, pads), [lo + d + hi for d, (lo, hi) in zip(shape, pads)]
    # broadcast a size-1 axis (or add a leading one)
    ns = [1] + list(shape) if 1 not in shape else list(shape)
    node = g.reshape(node, ns) if len(ns) != r else node
    tgt = [d if d != 1 else 1 + int(rng.integers(4)) for d in ns]
    return g.broadcast_to(node, tgt), tgt


def seed_shapes(rng, big: bool):
    a = 1 + int(rng.integers(5))
    shapes = [[a, 1 + int(rng.integers(5))], [1 + int(rng.integers(5)), 1 + int(rng.integers(5))],
              [1 + int(rng.integers(5)) for _ in range(1 + int(rng.integers(3)))]]
    if big:  # long last axes: vectorised loads, multi-wave lines
        shapes[2][-1] = int(rng.choice([64, 96, 130, 257, 1000]))
    return shapes


def _sixteenths(g: Graph, rng, shape, dt: DType):
    """A constant of multiples of 1/16 in [-1, 1] (exact in every float dtype)."""
    vals = (rng.integers(-16, 17, int(np.prod(shape))) / 16.0).astype(np.float32)
    node = g.constant_bytes(DType.F32, vals.tobytes(), list(shape))
    return node if dt == DType.F32 else g.cast(node, dt)


def _mfma_contraction(g: Graph, rng, dt: DType):
    """A contraction of length 64, 128 or 192 in one of four layouts; returns (node, shape)."""
    m, n, k = 1 + int(rng.integers(150)), 8 * (1 + int(rng.integers(40))), 64 * (1 + int(rng.integers(3)))
    kind = int(rng.integers(4))
    if kind == 0:  # [m, k] @ [k, n]
        return g.matmul(_sixteenths(g, rng, [m, k], dt), _sixteenths(g, rng, [k, n], dt)), [m, n]
    if kind == 1:  # [m, k] . [n, k]^T (the linear layout)
        return g.dot_general(_sixteenths(g, rng, [m, k], dt), _sixteenths(g, rng, [n, k], dt), [1], [1]), [m, n]
    if kind == 2:  # batched [b, m, k] @ [b, k, n]
        b = 1 + int(rng.integers(3))
        a, c = _sixteenths(g, rng, [b, m, k], dt), _sixteenths(g, rng, [b, k, n], dt)
        return g.dot_general(a, c, [2], [1], [0], [0]), [b, m, n]
    # transposed lhs: [k, m] contracted on its first axis
    return g.dot_general(_sixteenths(g, rng, [k, m], dt), _sixteenths(g, rng, [k, n], dt), [0], [0]), [m, n]


def _attention(g: Graph, rng, dt: DType):
    b, h, s = 1 + int(rng.integers(2)), 1 + int(rng.integers(3)), 1 + int(rng.integers(200))
    d = int(rng.choice([32, 64, 128]))
    q, k, v = (_sixteenths(g, rng, [b, h, s, d], dt) for _ in range(3))
    causal = bool(rng.integers(2))
    f = g.sdpa_fused if rng.integers(2) else g.sdpa_decomposed
    return f(q, k, v, causal)


def float_graph(seed: int, dt: DType):
    g, roots, _ = float_graph_info(seed, dt)
    return g, roots


def float_graph_info(seed: int, dt: DType):
    """(graph, roots, attn_roots): attn_roots are the roots that are attention outputs."""
    rng = np.random.default_rng([seed, int(dt), 7])
    g = Graph()
    nodes = [(_const(g, rng, s, dt), s) for s in seed_shapes(rng, seed % 3 == 0)]
    leaves = list(nodes)
    attn, mm = [], []
    for _ in range(8 + int(rng.integers(6))):
        node, shape = nodes[int(rng.integers(len(nodes)))]
        k = int(rng.integers(9))
        step = None
        if k == 7:
            step = _mfma_contraction(g, rng, dt)
            mm.append(step[0])
        elif k == 8:
            if len(attn) < 2:
                attn.append(_attention(g, rng, dt))
        elif k == 0:
            u = int(rng.integers(9))
            f = [g.neg, g.recip, g.sqrt, g.exp2, g.log2, g.sin, g.abs, g.floor, g.relu][u]
            step = (f(node), shape)
        elif k == 1:
            same = [n for n, s in nodes if s == shape]
            o = same[int(rng.integers(len(same)))]
            f = [g.add, g.mul, g.max, g.sub][int(rng.integers(4))]
            step = (f(node, o), shape)
        elif k == 2 and dt == DType.F32:
            mats = [(n, s) for n, s in nodes if len(s) == 2]
            if mats:
                an, ash = mats[int(rng.integers(len(mats)))]
                cands = [(n, s) for n, s in mats if s[0] == ash[1]]
                if cands:
                    bn, bsh = cands[int(rng.integers(len(cands)))]
                    step = (g.matmul(an, bn), [ash[0], bsh[1]])
        elif k == 3:
            ax = int(rng.integers(len(shape)))
            kind = int(rng.integers(3))
            if kind == 0:
                step = (g.sum(node, ax), shape[:ax] + shape[ax + 1:])
            elif kind == 1:
                step = (g.reduce_max(node, ax), shape[:ax] + shape[ax + 1:])
            else:
                step = (g.softmax(node, ax), shape)
        elif k == 4:
            to = FLOATS[int(rng.integers(len(FLOATS)))]
            step = (g.cast(g.cast(node, to), dt), shape)
        elif k == 5 and leaves:
            ln, ls = leaves[int(rng.integers(len(leaves)))]
            ax = int(rng.integers(len(ls)))
            step = (g.cast(g.argmax(ln, ax), dt), ls[:ax] + ls[ax + 1:])
        else:
            step = _movement(rng, g, node, shape)
        if step is not None and step[1] and all(d > 0 for d in step[1]):
            nodes.append(step)
    roots = [nodes[-1][0]] + [nodes[int(rng.integers(len(nodes)))][0] for _ in range(2)]
    return g, list(dict.fromkeys(roots + mm + attn)), set(attn)


def int_graph(seed: int, dt: DType):
    rng = np.random.default_rng([seed, int(dt), 11])
    g = Graph()
    nodes = [(_const(g, rng, s, dt), s) for s in seed_shapes(rng, seed % 3 == 0)]
    for _ in range(8 + int(rng.integers(6))):
        node, shape = nodes[int(rng.integers(len(nodes)))]
        k = int(rng.integers(4))
        if k == 0:
            same = [n for n, s in nodes if s == shape]
            o = same[int(rng.integers(len(same)))]
            f = [g.max, g.bit_and, g.bit_or, g.bit_xor, g.add][int(rng.integers(5))]
            step = (f(node, o), shape)
        elif k == 1:
            ax = int(rng.integers(len(shape)))
            kind = int(rng.integers(3))
            red = [g.reduce_max, g.sum, lambda n, a: g.cast(g.argmax(n, a), dt)][kind]
            step = (red(node, ax), shape[:ax] + shape[ax + 1:])
        else:
            step = _movement(rng, g, node, shape)
        if step[1] and all(d > 0 for d in step[1]):
            nodes.append(step)
    roots = [nodes[-1][0]] + [nodes[int(rng.integers(len(nodes)))][0] for _ in range(2)]
    return g, list(dict.fromkeys(roots))


def close_float(got: np.ndarray, want: np.ndarray, dt: DType) -> np.ndarray:
    """Elementwise agreement: NaN with NaN, same-signed overflow, else a relative band (f32
    1e-4 with a 1e-5 floor; 16-bit floats 2e-2 with a 2e-3 floor)."""
    got = got.astype(np.float64)
    want = want.astype(np.float64)
    rtol, atol = (1e-4, 1e-5) if dt == DType.F32 else (2e-2, 2e-3)
    both_nan = np.isnan(got) & np.isnan(want)
    big = (np.abs(got) > 1e30) & (np.abs(want) > 1e30) & (np.sign(got) == np.sign(want))
    with np.errstate(invalid="ignore"):
        ok = np.abs(got - want) <= atol + rtol * np.abs(want)
    return ok | both_nan | big
