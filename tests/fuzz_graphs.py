"""Seeded random graphs for differential testing (Differential.check's use,
lib/backend/differential.ml:80-88, over graphs no example spells out).

Each case draws a dtype, a shape (ragged sizes, rows of every template's
range), one or two params and a random element-wise expression over them,
then a root: a map, a reduction or scan (whole tensor or by rows), a
gather, a scatter_add, a broadcast or a matmul. Float inputs and
expressions stay positive and well scaled, so that sequential and tree
orders of summation agree to the 1e-4 band; integer expressions wrap and
must be bit-exact. Sizes stay small enough for the oracle to run in a
fraction of a second per case.
"""

from __future__ import annotations

import numpy as np

from cudacaml_amd import dsl as D
from cudacaml_amd.ir import F32, F64, I32, Graph

SIZES_1D = [1, 3, 63, 64, 255, 256, 257, 1000, 4096, 4097, 30001]
ROWS = [1, 2, 7, 64, 1024, 1100]
COLS = [1, 5, 63, 64, 65, 300, 1025, 2049]


def _float_expr(rng, leaves, depth):
    """A positive expression over positive leaves."""
    dt = leaves[0].dtype
    if depth == 0 or rng.random() < 0.3:
        return leaves[rng.integers(len(leaves))]
    k = rng.integers(8)
    a = _float_expr(rng, leaves, depth - 1)
    if k == 0:
        return D.add(a, _float_expr(rng, leaves, depth - 1))
    if k == 1:
        return D.mul(a, D.const(dt, float(rng.choice([0.5, 0.75, 1.25, 2.0]))))
    if k == 2:
        return D.max(a, _float_expr(rng, leaves, depth - 1))
    if k == 3:
        return D.min(a, _float_expr(rng, leaves, depth - 1))
    if k == 4:
        return D.sqrt(D.add(a, D.const(dt, 0.25)))
    if k == 5:
        return D.add(D.exp(D.neg(a)), D.const(dt, 0.5))
    if k == 6:
        b = _float_expr(rng, leaves, depth - 1)
        return D.select(D.lt(a, b), a, b)
    return D.mul(a, _float_expr(rng, leaves, depth - 1))


def _int_expr(rng, leaves, depth):
    if depth == 0 or rng.random() < 0.3:
        return leaves[rng.integers(len(leaves))]
    k = rng.integers(8)
    a = _int_expr(rng, leaves, depth - 1)
    c = lambda v: D.const(I32, int(v))  # noqa: E731
    if k == 0:
        return D.add(a, _int_expr(rng, leaves, depth - 1))
    if k == 1:
        return D.sub(a, _int_expr(rng, leaves, depth - 1))
    if k == 2:
        return D.mul(a, c(rng.integers(-7, 8)))
    if k == 3:
        return D.bit_xor(a, _int_expr(rng, leaves, depth - 1))
    if k == 4:
        return D.shr(a, c(rng.integers(0, 40)))
    if k == 5:
        return D.max(a, _int_expr(rng, leaves, depth - 1))
    if k == 6:
        return D.div(a, c(rng.choice([1, 3, -5, 7])))
    b = _int_expr(rng, leaves, depth - 1)
    return D.select(D.lt(a, b), a, b)


def _input(rng, dt, shape):
    if dt is I32:
        return rng.integers(-1000, 1000, size=shape, dtype=np.int64).astype(np.int32)
    return rng.uniform(0.5, 1.5, size=shape).astype(dt.np)


def case(seed):
    """(name, graph, inputs) for case `seed`."""
    rng = np.random.default_rng(1000 + seed)
    dt = [F32, F64, I32][rng.integers(3)]
    two_d = rng.random() < 0.5
    shape = (int(rng.choice(ROWS)), int(rng.choice(COLS))) if two_d else (int(rng.choice(SIZES_1D)),)
    n = int(np.prod(shape))
    if dt is F32 and n > (1 << 16):
        shape = (min(shape[0], 64), shape[1]) if two_d else (4097,)
        n = int(np.prod(shape))
    x = D.param("x", dt, shape)
    y = D.param("y", dt, shape)
    leaves = [x, y] if rng.random() < 0.6 else [x]
    if len(leaves) == 2:
        if dt is I32:
            body = lambda a, b: _int_expr(rng, [a, b], 3)  # noqa: E731
        else:
            body = lambda a, b: _float_expr(rng, [a, b], 3)  # noqa: E731
        m = D.map2(body, x, y)
    else:
        body = (lambda a: _int_expr(rng, [a], 3)) if dt is I32 else (lambda a: _float_expr(rng, [a], 3))
        m = D.map(body, x)
    inputs = [("x", _input(rng, dt, shape))]
    if len(leaves) == 2:
        inputs.append(("y", _input(rng, dt, shape)))
    zero = D.const(dt, 0.0 if dt is not I32 else 0)
    init = D.const(dt, float(rng.choice([0.0, 1.5])) if dt is not I32 else int(rng.choice([0, 3])))
    kind = rng.integers(9)
    if two_d and rng.random() < 0.25:
        kind = 3  # rows: the row templates (wave, block, split, row-sequential)
    outs = [("m", m)]
    if kind == 0:
        outs.append(("r", D.reduce(D.add, init, m)))
    elif kind == 1:
        outs.append(("r", D.reduce(D.max, D.const(dt, -1e30 if dt is not I32 else -(1 << 30)), m)))
    elif kind == 2:
        outs.append(("s", D.scan(D.add, init, m)))
    elif kind == 3 and two_d:
        outs.append(("rr", D.reduce_rows(D.add, init, m)))
        outs.append(("sr", D.scan_rows(D.max, zero, m)))
    elif kind == 4:
        k = int(rng.choice([1, 7, 1000, 5000]))
        idx = D.param("idx", I32, (k,))
        inputs.append(("idx", rng.integers(0, n, size=k).astype(np.int32)))
        outs.append(("g", D.gather(idx, D.flatten(m) if two_d else m)))
    elif kind == 5:
        bins = int(rng.choice([1, 17, 256, 8192, 20000]))
        idx = D.param("idx", I32, shape)
        inputs.append(("idx", rng.integers(0, bins, size=shape).astype(np.int32)))
        outs.append(("h", D.scatter_add(idx, m, (bins,))))
    elif kind == 6:
        s = D.reduce(D.add, zero, m)
        outs.append(("b", D.map2(lambda a, b: D.add(a, b), D.broadcast(shape, s), m)))
    elif kind == 7 and two_d and dt is not I32:
        kk = shape[1]
        w = D.param("w", dt, (kk, 17))
        inputs.append(("w", _input(rng, dt, (kk, 17))))
        outs.append(("mm", D.matmul(m, w)))
    else:
        outs.append(("t", D.map(lambda e: e, D.transpose(m))) if two_d else ("t", D.map(D.neg, m)))
    name = "fuzz%03d_%s_%s_%s" % (seed, dt.name, "x".join(map(str, shape)), outs[-1][0])
    return name, Graph.create("fuzz%d" % seed, outs), inputs
