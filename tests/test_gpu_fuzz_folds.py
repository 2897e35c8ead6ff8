"""Seeded random graphs for the two reduction paths that fold in a new
order: a whole-tensor reduction folded inside the map that writes its input
(the map's output is also a graph output, and the reduction is the next
root), and row reductions of rows of 1024 elements or more whose combine
allows any grouping (max, min; integer add, mul and bit operations; float
add and mul), folded as a tree. Random
dtypes, light element-wise expressions (tests/fuzz_graphs.py), ragged
sizes above the fold's 2^16 threshold and non-identity inits, against the
oracle under the per-output policy: integers and max/min bit-exact, float
sums within the accumulation band (row sums also against float64). A
whole-tensor float sum is held to the exact sum of its terms instead of the
oracle's: the interpreter's sequential f32 sum of a million terms or more
can itself leave the band (seed 81 of this generator, 1554799 terms: the
oracle 2.7e-4 from the exact sum, the device's tree 1.4e-6)."""

import math

import numpy as np
import pytest

import fuzz_graphs as FG
import oracle
from cudacaml_amd import backend_hip as H
from cudacaml_amd import differential as Diff
from cudacaml_amd import dsl as D
from cudacaml_amd.ir import F32, F64, I32, Graph

pytestmark = pytest.mark.gpu

N_CASES = 16
N_TREE_CASES = 24


def templates(g):
    return [l.split()[2] for l in H.plan(g).splitlines() if l.startswith("kernel")]


def folded_case(seed):
    r = np.random.default_rng(5000 + seed)
    dt = [F32, F64, I32][seed % 3]
    n = int(2 ** r.uniform(16.1, 21.5)) + int(r.integers(0, 4))
    x, y = D.param("x", dt, (n,)), D.param("y", dt, (n,))
    expr = FG._int_expr if dt is I32 else FG._float_expr
    m = D.map2(lambda a, b: expr(r, [a, b], 2), x, y)
    ops = ["add", "max", "min"] + (["mul", "xor"] if dt is I32 else [])
    op = ops[int(r.integers(len(ops)))]
    comb = {"add": D.add, "max": D.max, "min": D.min, "mul": D.mul, "xor": D.bit_xor}[op]
    iv = int(r.integers(-3, 4)) if dt is I32 else float(r.choice([0.0, 1.5, -2.0]))
    init = D.const(dt, iv)
    g = Graph.create("fold%d" % seed, [("m", m), ("s", D.reduce(comb, init, m))])
    inputs = [("x", FG._input(r, dt, (n,))), ("y", FG._input(r, dt, (n,)))]
    return g, inputs, (dt.name, n, op, iv)


def tree_case(seed):
    r = np.random.default_rng(6000 + seed)
    dt = [F32, F64, I32][seed % 3]
    rows, cols = int(r.choice([1024, 1100, 2048, 3001])), int(r.choice([1024, 1031, 2048, 2049, 5000]))
    x = D.param("x", dt, (rows, cols))
    ops = ["max", "min", "add", "mul"] + (["and"] if dt is I32 else [])
    op = ops[int(r.integers(len(ops)))]
    comb = {"add": D.add, "max": D.max, "min": D.min, "mul": D.mul, "and": D.bit_and}[op]
    iv = int(r.integers(-3, 4)) if dt is I32 else float(r.choice([0.0, 0.75, -1.0]))
    g = Graph.create("tree%d" % seed, [("s", D.reduce_rows(comb, D.const(dt, iv), x))])
    return g, [("x", FG._input(r, dt, (rows, cols)))], (dt.name, rows, cols, op, iv)


def _run(g, inputs):
    exp = oracle.run(g, inputs)
    c = H.compile(g)
    try:
        got = H.run(c, inputs)
    finally:
        c.release()
    return exp, got


@pytest.mark.parametrize("seed", list(range(N_CASES)) + [81])
def test_folded_reduction_fuzz(device, seed):
    g, inputs, what = folded_case(seed)
    print("case", seed, *what, flush=True)
    t = templates(g)
    assert "reduce_split" not in t and "reduce_split_fold" in t, (what, t)
    exp, got = _run(g, inputs)
    float_sum = what[0] != "i32" and what[2] == "add"
    bad = [v for v in Diff.policy_check(g, exp, got) if not v.ok and not (float_sum and v.name == "s")]
    assert not bad, (what, bad)
    if float_sum:
        e, d = dict(exp), dict(got)
        exact = math.fsum([float(what[3])] + e["m"].astype(np.float64).tolist())
        tol = 1e-4 if what[0] == "f32" else 1e-12
        err = abs(float(d["s"]) - exact)
        assert err <= tol * (1 + abs(exact)), (what, float(d["s"]), exact, float(e["s"]))


@pytest.mark.parametrize("seed", range(N_TREE_CASES))
def test_tree_row_reduction_fuzz(device, seed):
    g, inputs, what = tree_case(seed)
    print("case", seed, *what, flush=True)
    assert "reduce_rowseq" not in templates(g), what
    exp, got = _run(g, inputs)
    if what[0] != "i32" and what[3] in ("add", "mul"):
        bad = [v for v in Diff.policy_check(g, exp, got) if not v.ok]
        assert not bad, (what, bad)
        if what[3] == "mul":
            return
        e64 = inputs[0][1].astype(np.float64).sum(axis=1) + what[4]
        d = np.asarray(got[0][1], dtype=np.float64)
        assert np.all(np.abs(d - e64) <= 1e-4 * (1 + np.abs(e64))), what
        return
    for (name, e), (_, d) in zip(exp, got):
        # any grouping gives the same bits (no NaN among these inputs)
        np.testing.assert_array_equal(e.view(np.uint8), d.view(np.uint8), err_msg=str(what))


def scan_case(seed):
    r = np.random.default_rng(7000 + seed)
    dt = [F32, F64, I32][seed % 3]
    rows, cols = int(r.choice([1024, 1100])), int(r.choice([2048, 2049, 5000, 9001, 30000]))
    x = D.param("x", dt, (rows, cols))
    ops = ["max", "min", "add", "mul"] + (["xor"] if dt is I32 else [])
    op = ops[int(r.integers(len(ops)))]
    comb = {"add": D.add, "max": D.max, "min": D.min, "mul": D.mul, "xor": D.bit_xor}[op]
    iv = int(r.integers(-3, 4)) if dt is I32 else float(r.choice([0.0, 0.75, -1.0]))
    g = Graph.create("tscan%d" % seed, [("p", D.scan_rows(comb, D.const(dt, iv), x))])
    return g, [("x", FG._input(r, dt, (rows, cols)))], (dt.name, rows, cols, op, iv)


@pytest.mark.parametrize("seed", range(N_CASES))
def test_tile_row_scan_fuzz(device, seed):
    """Scans of 1024 rows or more of 2048 elements or more, whose combine
    allows any grouping, run as tile scans (a workgroup a row, or a
    look-back chain of tiles): integers, max and min bit-exact against the
    oracle; float add and mul within the policy's band, add also against
    the float64 prefix sums."""
    g, inputs, what = scan_case(seed)
    print("case", seed, *what, flush=True)
    t = templates(g)
    assert "scan_rowseq" not in t and ("scan_tile" in t or "scan_lookback" in t), (what, t)
    exp, got = _run(g, inputs)
    if what[0] != "i32" and what[3] in ("add", "mul"):
        bad = [v for v in Diff.policy_check(g, exp, got) if not v.ok]
        assert not bad, (what, bad)
        if what[3] == "add":
            e64 = np.cumsum(inputs[0][1].astype(np.float64), axis=1) + what[4]
            d = np.asarray(got[0][1], dtype=np.float64)
            assert np.all(np.abs(d - e64) <= 1e-4 * (1 + np.abs(e64))), what
        return
    for (name, e), (_, d) in zip(exp, got):
        np.testing.assert_array_equal(e.view(np.uint8), d.view(np.uint8), err_msg=str(what))


N_EXPR_CASES = 24


def expr_folded_case(seed):
    """m = a map of x and y (an output); s = a reduction of an element-wise
    expression of m and z, and in some cases of a gather of z, a scalar, or
    of an f64 tensor cast down; m 1-D or 2-D (s reads it flattened); in
    some cases another root between m and s. Returns the graph, the graph
    with the expression as its output (for the exact float sum), inputs
    and a description."""
    r = np.random.default_rng(8000 + seed)
    dt = [F32, F64, I32][seed % 3]
    n = int(2 ** r.uniform(16.1, 21)) + int(r.integers(0, 4))
    two_d = r.random() < 0.35
    shape = (int(r.choice([64, 257])), 0) if two_d else (n,)
    if two_d:
        shape = (shape[0], max(1, n // shape[0]))
        n = shape[0] * shape[1]
    expr = FG._int_expr if dt is I32 else FG._float_expr
    x, y, z = D.param("x", dt, shape), D.param("y", dt, shape), D.param("z", dt, shape)
    inputs = [("x", FG._input(r, dt, shape)), ("y", FG._input(r, dt, shape)), ("z", FG._input(r, dt, shape))]
    m = D.map2(lambda a, b: expr(r, [a, b], 2), x, y)
    extra = str(r.choice(["plain", "gather", "scalar", "cast", "between", "unread"]))
    # unread: m is no output, only the expression reads it (twice, so the
    # plan materialises it), and its kernel stores nothing but the partials
    outs = [] if extra == "unread" else [("m", m)]
    if extra == "between":
        outs.append(("u", D.map(lambda a: D.add(a, a), x)))
    e = D.map2(lambda a, c: expr(r, [a, c], 2), m, z)
    if extra == "unread":
        e = D.map2(lambda u, v: D.add(u, v), e, m)
    flat = D.flatten(e) if two_d else e
    if extra == "gather":
        idx = D.param("idx", I32, (n,))
        inputs.append(("idx", r.integers(0, n, size=n).astype(np.int32)))
        flat = D.map2(lambda a, v: D.max(a, v), flat, D.gather(idx, D.flatten(z) if two_d else z))
    elif extra == "scalar":
        k = D.scalar("k", dt)
        inputs.append(("k", np.array(3 if dt is I32 else 1.25, dtype=dt.np)))
        flat = D.map2(lambda a, v: D.mul(a, v), flat, D.broadcast((n,), k))
    elif extra == "cast":
        w = D.param("w", F64 if dt is not F64 else F32, (n,))
        inputs.append(("w", r.uniform(0.5, 1.5, size=n).astype(w.dtype.np)))
        flat = D.map2(lambda a, v: D.add(a, D.cast(dt, v)), flat, w)
    ops = ["add", "max", "min"] + (["mul", "xor"] if dt is I32 else [])
    op = ops[int(r.integers(len(ops)))]
    comb = {"add": D.add, "max": D.max, "min": D.min, "mul": D.mul, "xor": D.bit_xor}[op]
    iv = int(r.integers(-3, 4)) if dt is I32 else float(r.choice([0.0, 1.5, -2.0]))
    s = D.reduce(comb, D.const(dt, iv), flat)
    g = Graph.create("efold%d" % seed, outs + [("s", s)])
    g_terms = Graph.create("eterms%d" % seed, [("e", flat)])
    knobs = "map_unroll=2" if seed % 4 == 3 else ""
    return g, g_terms, inputs, (dt.name, shape, extra, op, iv, knobs)


@pytest.mark.parametrize("seed", range(N_EXPR_CASES))
def test_expression_fold_fuzz(device, monkeypatch, seed):
    """A whole-tensor reduction of an element-wise expression of a map's
    output folds inside that map's kernel: integers, max and min bit-exact
    against the oracle; a float sum within the band of the exact sum of
    its terms (the oracle's own terms, which the device's map matches)."""
    g, g_terms, inputs, what = expr_folded_case(seed)
    print("case", seed, *what, flush=True)
    if what[5]:
        monkeypatch.setenv("CCHIP_TUNE", what[5])
    t = templates(g)
    assert "reduce_split" not in t and "reduce_split_fold" in t, (what, t)
    if what[2] == "unread":
        assert " elided" in H.plan(g), what
    exp, got = _run(g, inputs)
    float_sum = what[0] != "i32" and what[3] == "add"
    bad = [v for v in Diff.policy_check(g, exp, got) if not v.ok and not (float_sum and v.name == "s")]
    assert not bad, (what, bad)
    e, d = dict(exp), dict(got)
    if not float_sum:
        np.testing.assert_array_equal(np.atleast_1d(e["s"]).view(np.uint8), np.atleast_1d(d["s"]).view(np.uint8),
                                      err_msg=str(what))
        return
    names = {n for n, _ in g_terms.params}
    terms = dict(oracle.run(g_terms, [(k, v) for k, v in inputs if k in names]))["e"]
    exact = math.fsum([float(what[4])] + terms.astype(np.float64).tolist())
    tol = 1e-4 if what[0] == "f32" else 1e-12
    assert abs(float(d["s"]) - exact) <= tol * (1 + abs(exact)), (what, float(d["s"]), exact, float(e["s"]))


def test_expression_fold_reports_index_errors(device):
    """A sum of an expression that gathers, folded inside the map that
    writes its operand: an index out of range is reported as the unfused
    reduction reports it, and the next run with good indices is clean and
    matches the oracle."""
    n = (1 << 18) + 3
    x, z = D.param("x", F32, (n,)), D.param("z", F32, (n,))
    idx = D.param("idx", I32, (n,))
    a = D.map(lambda v: D.add(v, D.const(F32, 0.5)), x)
    s = D.reduce(D.max, D.const(F32, -1e30), D.map2(D.mul, a, D.gather(idx, z)))
    g = Graph.create("eerr", [("a", a), ("s", s)])
    t = templates(g)
    assert "reduce_split" not in t and "reduce_split_fold" in t, t
    r = np.random.default_rng(9)
    good = r.integers(0, n, size=n).astype(np.int32)
    bad = good.copy()
    bad[n // 2] = n
    base = [("x", r.uniform(-1, 1, n).astype(np.float32)), ("z", r.uniform(-1, 1, n).astype(np.float32))]
    c = H.compile(g)
    try:
        with pytest.raises(ValueError, match="gather index out of bounds"):
            H.run(c, base + [("idx", bad)])
        got = dict(H.run(c, base + [("idx", good)]))
    finally:
        c.release()
    exp = dict(oracle.run(g, base + [("idx", good)]))
    for k in exp:
        np.testing.assert_array_equal(np.atleast_1d(got[k]).view(np.uint8), np.atleast_1d(exp[k]).view(np.uint8))
