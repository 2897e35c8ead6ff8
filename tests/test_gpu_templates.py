"""Each Reduce/Scan/Map/Scatter template variant on the device, chosen
through the shapes that select it (the plan records which one ran), against
the oracle: integer results bit-exact, float results to the policy bar.
Ragged sizes (not multiples of 4, of a tile, of a workgroup) and empty
rows are included, as the reference tests them (test_system.ml:123-128)."""

import numpy as np
import pytest

import oracle
from cudacaml_amd import backend_hip as H
from cudacaml_amd import differential as Diff
from cudacaml_amd import dsl as D
from cudacaml_amd.examples import configs as C
from cudacaml_amd.ir import F32, F64, I32, I64, Graph

pytestmark = pytest.mark.gpu


def templates(g):
    return [l.split()[2] for l in H.plan(g).splitlines() if l.startswith("kernel")]


def data(dtype, shape, seed):
    n = int(np.prod(shape))
    if dtype is I32:
        return C.small_ints(seed, shape)
    if dtype is I64:
        return (C.small_ints(seed, (n,)).astype(np.int64) * 123456789 - 987654321).reshape(shape)
    return C.uniform_pm1(seed, shape).astype(dtype.np)


def check(g, inputs, expect_templates):
    got_t = templates(g)
    for t in expect_templates:
        assert t in got_t, (t, got_t)
    exp = oracle.run(g, inputs)
    c = H.compile(g)
    try:
        got = H.run(c, inputs)
    finally:
        c.release()
    bad = [v for v in Diff.policy_check(g, exp, got) if not v.ok]
    assert not bad, bad


SCAN_CASES = [
    # (rows, len, dtype, template)
    (100, 37, I32, "scan_wave"),
    (100, 64, F32, "scan_wave"),
    (7, 1, I64, "scan_wave"),
    (300, 1000, I32, "scan_tile"),
    (200, 4097, I64, "scan_tile"),
    (3, 8192, F64, "scan_tile"),
    (1, 1 << 20, I32, "scan_lookback"),
    (5, 300001, I32, "scan_lookback"),
    (8, 100003, F64, "scan_lookback"),
    (2, 77777, I64, "scan_lookback"),
    (1024, 333, I32, "scan_rowseq"),
    (2048, 64, F32, "scan_rowseq"),
    (1500, 2050, I64, "scan_rowseq"),
]


@pytest.mark.parametrize("rows,n,dtype,tpl", SCAN_CASES, ids=lambda v: str(v))
def test_scan_variants(device, rows, n, dtype, tpl):
    x = D.param("x", dtype, (rows, n))
    g = Graph.create("scan", [("p", D.scan_rows(D.add, D.const(dtype, 0), x))])
    check(g, [("x", data(dtype, (rows, n), 11))], [tpl])


REDUCE_CASES = [
    (100, 37, I32, "reduce_wave"),
    (300, 2048, F32, "reduce_wave"),
    (600, 4096, I32, "reduce_block"),
    (700, 3001, F64, "reduce_block"),
    (1, 1 << 22, I32, "reduce_split"),
    (3, 999999, I64, "reduce_split"),
    (200, 8192, F32, "reduce_split"),
    (1024, 333, I32, "reduce_rowseq"),
    (4096, 5000, F64, "reduce_rowseq"),
]


@pytest.mark.parametrize("rows,n,dtype,tpl", REDUCE_CASES, ids=lambda v: str(v))
def test_reduce_variants(device, rows, n, dtype, tpl):
    x = D.param("x", dtype, (rows, n))
    z = D.const(dtype, 0)
    g = Graph.create("red", [("s", D.reduce_rows(D.add, z, x)),
                             ("m", D.reduce_rows(D.max, D.const(dtype, -(1 << 30)), x))])
    check(g, [("x", data(dtype, (rows, n), 12))], [tpl])


def test_reduce_empty_rows(device):
    x = D.param("x", F32, (5, 0))
    g = Graph.create("e", [("s", D.reduce_rows(D.add, D.const(F32, 2.5), x))])
    check(g, [("x", np.zeros((5, 0), np.float32))], ["reduce_empty"])


def test_scan_rows_exact_order_f32(device):
    """Row-sequential scans fold in the interpreter's order: bit-exact f32."""
    x = D.param("x", F32, (2048, 3000))
    g = Graph.create("s", [("p", D.scan_rows(D.add, D.const(F32, 0.0), x)),
                           ("s", D.reduce_rows(D.add, D.const(F32, 0.0), x))])
    v = data(F32, (2048, 3000), 13)
    exp = oracle.run(g, [("x", v)])
    c = H.compile(g)
    got = H.run(c, [("x", v)])
    c.release()
    for (n, e), (_, gv) in zip(exp, got):
        np.testing.assert_array_equal(e, gv, err_msg=n)


@pytest.mark.parametrize("n", [0, 1, 3, 4, 5, 1023, 1025, 65537])
def test_map_ragged(device, n):
    x = D.param("x", F32, (n,))
    y = D.param("y", I32, (n,))
    g = Graph.create("m", [("r", D.map2(lambda a, b: D.mul(a, D.cast(F32, b)), x, y)),
                           ("q", D.map(lambda b: D.shr(D.mul(b, D.const(I32, -7)), D.const(I32, 3)), y))])
    check(g, [("x", data(F32, (n,), 1)), ("y", data(I32, (n,), 2))], [] if n == 0 else ["map"])


@pytest.mark.parametrize("dtype", [F32, F64, I32])
def test_scatter_dtypes(device, dtype):
    n, bins = 100003, 1000
    idx = D.param("idx", I32, (n,))
    src = D.param("src", dtype, (n,))
    g = Graph.create("h", [("h", D.scatter_add(idx, src, (bins,)))])
    check(g, [("idx", C.bin_indices(3, n, bits=10) % bins), ("src", data(dtype, (n,), 4))],
          ["scatter_zero", "scatter_atomic"])


def test_gather_out_of_range_raises(device):
    x = D.param("x", F32, (3,))
    i = D.param("i", I32, (4,))
    c = H.compile(Graph.create("g", [("r", D.gather(i, x))]))
    with pytest.raises(ValueError, match="gather index out of bounds"):
        H.run(c, [("x", np.ones(3, np.float32)), ("i", np.array([0, 1, 3, 2], np.int32))])
    # The error word is cleared: a good run afterwards succeeds.
    r = H.run(c, [("x", np.array([1, 2, 3], np.float32)), ("i", np.array([2, 1, 0, 2], np.int32))])
    assert r[0][1].tolist() == [3, 2, 1, 3]
    c.release()


def test_scatter_out_of_range_raises(device):
    i = D.param("i", I32, (4,))
    s = D.param("s", I32, (4,))
    c = H.compile(Graph.create("h", [("h", D.scatter_add(i, s, (4,)))]))
    with pytest.raises(ValueError, match="scatter_add index out of bounds"):
        H.run(c, [("i", np.array([0, 1, -1, 2], np.int32)), ("s", np.ones(4, np.int32))])
    c.release()
