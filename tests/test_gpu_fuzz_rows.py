"""Seeded random graphs for the row paths that let one root's kernel serve
another root's reads:

- gathers of every row's last element (index p * L + L - 1), which read a
  side buffer that the row scan (one lane a row) or the map root writes,
  one value a row: the Monte Carlo pricer's final prices. Each case mixes
  in what must not take that path: a gather of another column, another
  tensor of the same shape read at the gathered index, and a second row
  scan of another row length read through a reshape (its own side buffer
  is for its own rows);
- row scans that take the one-workgroup-a-row tile template, fused with
  the tree reductions of the same rows into one kernel: config 2's scan,
  sum and max.

Random dtypes, combines, inits, ragged rows and light element-wise
expressions (tests/fuzz_graphs.py), against the oracle under the
per-output policy: integers, max and min bit-exact, float sums within the
accumulation band."""

import numpy as np
import pytest

import fuzz_graphs as FG
import oracle
from cudacaml_amd import backend_hip as H
from cudacaml_amd import differential as Diff
from cudacaml_amd import dsl as D
from cudacaml_amd.ir import F32, F64, I32, Graph

pytestmark = pytest.mark.gpu

N_ROWLAST_CASES = 16
N_SIBLING_CASES = 16

COMBINES = {"add": D.add, "max": D.max, "min": D.min}


def _init(r, dt):
    return D.const(dt, int(r.integers(-3, 4)) if dt is I32 else float(r.choice([0.0, 0.5, -1.0])))


def _expr(r, dt):
    return FG._int_expr if dt is I32 else FG._float_expr


def rowlast_case(seed):
    r = np.random.default_rng(7000 + seed)
    dt = [F32, F64, I32][seed % 3]
    rows = int(r.choice([1024, 1031, 2048, 3001]))
    L = int(r.choice([2, 3, 64, 65, 100, 334, 1000]))
    expr = _expr(r, dt)
    x = D.param("x", dt, (rows, L))
    inputs = [("x", FG._input(r, dt, (rows, L)))]
    outs = []
    src_kind = ["scan", "map"][int(r.integers(2))]
    op = str(r.choice(list(COMBINES)))
    if src_kind == "scan":
        p = D.scan_rows(COMBINES[op], _init(r, dt), D.map(lambda a: expr(r, [a], 2), x))
    else:
        # a materialised map root (it is an output too)
        p = D.map(lambda a: expr(r, [a], 2), x)
        outs.append(("p", p))
    mix = ["none", "param", "reshaped_scan"][int(r.integers(3))]
    src = p
    if mix == "param":
        y = D.param("y", dt, (rows, L))
        inputs.append(("y", FG._input(r, dt, (rows, L))))
        src = D.map2(lambda a, b: expr(r, [a, b], 2), p, y)
    elif mix == "reshaped_scan" and L % 2 == 0:
        # a second row scan of rows half as long, with its own row-last
        # gather (so its own side buffer), read through a reshape
        z = D.param("z", dt, (2 * rows, L // 2))
        inputs.append(("z", FG._input(r, dt, (2 * rows, L // 2))))
        q = D.scan_rows(D.max, _init(r, dt), z)
        iq = D.map(lambda i: D.add(D.mul(i, D.const(I32, L // 2)), D.const(I32, L // 2 - 1)), D.iota((2 * rows,)))
        outs.append(("qlast", D.gather(iq, q)))
        src = D.map2(D.add, p, D.reshape((rows, L), q))
    else:
        mix = "none"
    col = L - 1 if r.random() < 0.75 else int(r.integers(L))
    idx = D.map(lambda i: D.add(D.mul(i, D.const(I32, L)), D.const(I32, col)), D.iota((rows,)))
    last = D.gather(idx, D.map(lambda a: D.mul(a, D.const(dt, 3)), src))
    outs.append(("last", last))
    if r.random() < 0.5:
        outs.append(("s", D.reduce(D.add, D.const(dt, 0), last)))
    g = Graph.create("rowlast%d" % seed, outs)
    return g, inputs, (dt.name, rows, L, src_kind, op, mix, col)


def sibling_case(seed):
    r = np.random.default_rng(8000 + seed)
    dt = [F32, F64, I32][seed % 3]
    if r.random() < 0.5:
        rows, cols = int(r.choice([1, 7, 64, 300])), int(r.choice([65, 300, 1025, 4096, 9001]))
    else:
        rows, cols = int(r.choice([1024, 1100])), int(r.choice([2048, 2049, 4000]))
    expr = _expr(r, dt)
    x = D.param("x", dt, (rows, cols))
    m = D.map(lambda a: expr(r, [a], 2), x) if r.random() < 0.7 else x
    sop = str(r.choice(list(COMBINES)))
    roots = [("scan", D.scan_rows(COMBINES[sop], _init(r, dt), m))]
    ops = []
    for k in range(int(r.integers(1, 4))):
        op = str(r.choice(list(COMBINES)))
        ops.append(op)
        roots.append(("red%d" % k, D.reduce_rows(COMBINES[op], _init(r, dt), m)))
    order = r.permutation(len(roots))
    outs = [roots[i] for i in order]
    if r.random() < 0.4:
        # a consumer of the first root in the plan, after it
        first = outs[0][1]
        outs.append(("after", D.map(lambda a: D.add(a, D.const(dt, 1)), first)))
    g = Graph.create("sib%d" % seed, outs)
    inputs = [("x", FG._input(r, dt, (rows, cols)))]
    return g, inputs, (dt.name, rows, cols, sop, ops, [outs[i][0] for i in range(len(outs))])


def _check(g, inputs, what):
    exp = oracle.run(g, inputs)
    c = H.compile(g)
    try:
        got = H.run(c, inputs)
    finally:
        c.release()
    bad = [v for v in Diff.policy_check(g, exp, got) if not v.ok]
    assert not bad, (what, bad)


@pytest.mark.parametrize("seed", range(N_ROWLAST_CASES))
def test_row_last_gather_fuzz(device, seed):
    g, inputs, what = rowlast_case(seed)
    print("case", seed, *what, flush=True)
    _check(g, inputs, what)


@pytest.mark.parametrize("seed", range(N_SIBLING_CASES))
def test_sibling_rows_fuzz(device, seed):
    g, inputs, what = sibling_case(seed)
    print("case", seed, *what, flush=True)
    _check(g, inputs, what)
