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
from cudacaml_amd.examples import black_scholes as bs
from cudacaml_amd.examples import configs as C
from cudacaml_amd.examples import programs as P
from cudacaml_amd.examples import refbench as RB
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
    # tile boundaries: 26624 elements a tile for 4-byte values, 16384 for
    # 8-byte ones (one tile and one element; exactly two tiles)
    (2, 26625, I32, "scan_lookback"),
    (3, 53248, I32, "scan_lookback"),
    (2, 16385, I64, "scan_lookback"),
    (3, 32768, F64, "scan_lookback"),
    # 1024 rows or more, one lane a row in order (run with rs_tree=0, so at
    # every length)
    (1024, 333, I32, "scan_rowseq"),
    (2048, 64, F32, "scan_rowseq"),
    (1500, 2050, I64, "scan_rowseq"),
    # four tiles a row or more: one wave folds while four load and store
    # (ragged last tiles; a last workgroup with rows past the end)
    (1024, 20003, F32, "scan_rowseq"),
    (1030, 9000, I32, "scan_rowseq"),
    (2048, 9001, F64, "scan_rowseq"),
    # 1024 rows or more of 2048 elements or more (the default): a workgroup
    # a row, or a look-back chain of tiles a row
    (1500, 2050, I64, "scan_tile"),
    (1030, 9000, I32, "scan_tile"),
    (2048, 9001, F64, "scan_tile"),
    (1024, 20003, F32, "scan_tile"),
    (1024, 40000, I32, "scan_lookback"),
    (1024, 30000, F32, "scan_lookback"),
]


def check_scans(monkeypatch, g, inputs, tpl, init):
    """check() for an add scan "p" (and a max scan "q"). The scan_rowseq
    cases run with rs_tree=0, so the in-order template is the one under
    test at every length. A float add scan through a tile template is
    checked against the float64 prefix sums plus init, within the policy's
    band: over long rows the interpreter's own in-order f32 prefix drifts
    beyond the band where a prefix is near zero. Everything else against
    the oracle."""
    if tpl == "scan_rowseq":
        monkeypatch.setenv("CCHIP_TUNE", "rs_tree=0")
    assert tpl in templates(g), (tpl, templates(g))
    exp = oracle.run(g, inputs)
    c = H.compile(g)
    try:
        got = H.run(c, inputs)
    finally:
        c.release()
    x = inputs[0][1]
    fl = x.dtype.kind == "f" and tpl != "scan_rowseq"
    bad = [v for v in Diff.policy_check(g, exp, got) if not v.ok and not (fl and v.name == "p")]
    assert not bad, bad
    if fl:
        p = np.asarray(dict(got)["p"], dtype=np.float64)
        e = np.cumsum(x.astype(np.float64), axis=1) + init
        assert np.max(np.abs(p - e) / (1 + np.abs(e))) <= (1e-4 if x.dtype == np.float32 else 1e-12)


@pytest.mark.parametrize("rows,n,dtype,tpl", SCAN_CASES, ids=lambda v: str(v))
def test_scan_variants(device, monkeypatch, rows, n, dtype, tpl):
    x = D.param("x", dtype, (rows, n))
    g = Graph.create("scan", [("p", D.scan_rows(D.add, D.const(dtype, 0), x))])
    check_scans(monkeypatch, g, [("x", data(dtype, (rows, n), 11))], tpl, 0)


REDUCE_CASES = [
    (100, 37, I32, "reduce_wave"),
    (300, 2048, F32, "reduce_wave"),
    (600, 4096, I32, "reduce_block"),
    (700, 3001, F64, "reduce_block"),
    (1, 1 << 22, I32, "reduce_split"),
    (3, 999999, I64, "reduce_split"),
    (200, 8192, F32, "reduce_split"),
    # 1024 rows or more: short rows one lane a row, in order
    (1024, 333, F32, "reduce_rowseq"),
    (4096, 500, F64, "reduce_rowseq"),
    (1024, 333, I32, "reduce_rowseq"),
    # rows of 1024 or more elements: a tree, a wave or a workgroup a row
    (1024, 1500, I32, "reduce_wave"),
    (2048, 2048, F32, "reduce_wave"),
    (1030, 30000, I32, "reduce_block"),
    (4096, 5000, F64, "reduce_block"),
    (1024, 20003, F32, "reduce_block"),
]


def check_rows(g, inputs, tpl, init):
    """check() for a row sum "s" and a row max "m": a float sum against the
    float64 row sums plus init, within the policy's band, everything else
    against the oracle. Over rows of 20003 elements the interpreter's own
    in-order f32 fold drifts by up to 3e-4 from the exact sum, beyond the
    band where a row sums to near zero, so it is not the yardstick for a
    tree's sum there."""
    assert tpl in templates(g), (tpl, templates(g))
    exp = oracle.run(g, inputs)
    c = H.compile(g)
    try:
        got = H.run(c, inputs)
    finally:
        c.release()
    x = inputs[0][1]
    fl = x.dtype.kind == "f"
    bad = [v for v in Diff.policy_check(g, exp, got) if not v.ok and not (fl and v.name == "s")]
    assert not bad, bad
    if fl:
        s = np.asarray(dict(got)["s"], dtype=np.float64)
        e = x.astype(np.float64).sum(axis=1) + init
        assert np.max(np.abs(s - e) / (1 + np.abs(e))) <= (1e-4 if x.dtype == np.float32 else 1e-12)


@pytest.mark.parametrize("rows,n,dtype,tpl", REDUCE_CASES, ids=lambda v: str(v))
def test_reduce_variants(device, rows, n, dtype, tpl):
    x = D.param("x", dtype, (rows, n))
    z = D.const(dtype, 0)
    g = Graph.create("red", [("s", D.reduce_rows(D.add, z, x)),
                             ("m", D.reduce_rows(D.max, D.const(dtype, -(1 << 30)), x))])
    check_rows(g, [("x", data(dtype, (rows, n), 12))], tpl, 0)


@pytest.mark.parametrize("rows,n,dtype,tpl", REDUCE_CASES, ids=lambda v: str(v))
def test_reduce_init_applied_once(device, rows, n, dtype, tpl):
    """init is not the identity here: the interpreter folds it in once per
    row (R2), so a template that seeded every lane with it would be off by
    (lanes - 1) * init."""
    x = D.param("x", dtype, (rows, n))
    g = Graph.create("red", [("s", D.reduce_rows(D.add, D.const(dtype, 5), x)),
                             ("m", D.reduce_rows(D.max, D.const(dtype, 3), x))])
    check_rows(g, [("x", data(dtype, (rows, n), 14))], tpl, 5)


@pytest.mark.parametrize("rows,n,dtype,tpl", SCAN_CASES, ids=lambda v: str(v))
def test_scan_init_applied_once(device, monkeypatch, rows, n, dtype, tpl):
    x = D.param("x", dtype, (rows, n))
    g = Graph.create("scan", [("p", D.scan_rows(D.add, D.const(dtype, 7), x)),
                              ("q", D.scan_rows(D.max, D.const(dtype, 2), x))])
    check_scans(monkeypatch, g, [("x", data(dtype, (rows, n), 15))], tpl, 7)


SIBLING_CASES = [
    # (rows, len, dtype): ragged rows (not a multiple of 4: scalar loads),
    # short rows (the reductions alone would take reduce_wave), 1024 rows
    # or more, the longest one-tile rows (26624 elements of 4 bytes, 16384
    # of 8 bytes)
    (600, 3001, F32),
    (300, 100, F32),
    (1030, 9000, I32),
    (2000, 2048, I64),
    (513, 26624, I32),
    (700, 16384, F64),
    (257, 26623, F32),
]


def sibling_graph(dtype, rows, n):
    """A row scan and three row reductions of the same tensor, with
    non-identity inits: config 2's shape, plus min."""
    x = D.param("x", dtype, (rows, n))
    lo = -(1 << 30) if dtype.name in ("i32", "i64") else -1e30
    return Graph.create("sib", [("s", D.reduce_rows(D.add, D.const(dtype, 5), x)),
                                ("m", D.reduce_rows(D.max, D.const(dtype, lo), x)),
                                ("p", D.scan_rows(D.add, D.const(dtype, 7), x)),
                                ("n", D.reduce_rows(D.min, D.const(dtype, 3), x))])


def check_siblings(g, inputs, init_s, init_p):
    """Integer outputs, max and min against the oracle bit for bit; a float
    sum and prefix sum against float64 within the policy's band (the
    interpreter's in-order f32 folds drift beyond it over long rows)."""
    exp = dict(oracle.run(g, inputs))
    c = H.compile(g)
    try:
        got = dict(H.run(c, inputs))
    finally:
        c.release()
    x = inputs[0][1]
    fl = x.dtype.kind == "f"
    for name in ("m", "n") if fl else ("s", "m", "p", "n"):
        np.testing.assert_array_equal(got[name], exp[name], err_msg=name)
    if fl:
        tol = 1e-4 if x.dtype == np.float32 else 1e-12
        x64 = x.astype(np.float64)
        e = x64.sum(axis=1) + init_s
        assert np.max(np.abs(got["s"] - e) / (1 + np.abs(e))) <= tol
        e = np.cumsum(x64, axis=1) + init_p
        assert np.max(np.abs(got["p"] - e) / (1 + np.abs(e))) <= tol
    return got


@pytest.mark.parametrize("rows,n,dtype", SIBLING_CASES, ids=lambda v: str(v))
def test_sibling_row_roots_one_kernel(device, monkeypatch, rows, n, dtype):
    """The row scan and the reductions of the same tensor in one kernel
    (each row read once), against the oracle; then the same graph with
    sibling_fuse=0 (each root its own kernels): integer results equal bit
    for bit."""
    g = sibling_graph(dtype, rows, n)
    assert templates(g) == ["scan_tile_fold"], templates(g)
    ins = [("x", data(dtype, (rows, n), 61))]
    got = check_siblings(g, ins, 5, 7)
    monkeypatch.setenv("CCHIP_TUNE", "sibling_fuse=0")
    assert "scan_tile_fold" not in templates(g)
    sep = check_siblings(g, ins, 5, 7)
    for name in ("m", "n") if dtype in (F32, F64) else ("s", "m", "p", "n"):
        np.testing.assert_array_equal(got[name], sep[name], err_msg=name)


def test_sibling_group_runs_before_a_consumer_of_its_first_root(device):
    """The group's kernel runs where its first root stands in the plan: a
    root between the reduction and the scan reads the reduction's output,
    and a map read twice (materialised) is the shared tensor."""
    rows, n = 700, 5000
    x = D.param("x", F32, (rows, n))
    m = D.map(lambda v: D.add(D.mul(v, v), D.const(F32, 0.25)), x)
    s = D.reduce_rows(D.max, D.const(F32, 0.0), m)
    t = D.map(lambda v: D.mul(v, D.const(F32, 3.0)), s)
    p = D.scan_rows(D.max, D.const(F32, -1.0), m)
    g = Graph.create("sib2", [("s", s), ("t", t), ("p", p)])
    assert templates(g) == ["map", "scan_tile_fold", "map"], templates(g)
    check(g, [("x", data(F32, (rows, n), 62))], ["scan_tile_fold"])


SPLIT8_CASES = [
    # (rows, len, dtype, combine, knobs): row-sequential scans of 8-byte
    # values with split roles (four tiles a row or more), by default
    # (rows shorter than the tile scans' 2048) and with the in-order and
    # plain-store knobs; the case a random-knob search found wrong before
    # the loaders' stores kept to their own groups
    (4096, 1000, F64, "add", ""),
    (4096, 1000, I64, "add", ""),
    (1100, 4000, F64, "min", "rs_tree=0,rs_nt=0"),
    (2048, 3000, F64, "add", "rs_tree=0"),
    (1030, 5000, I64, "max", "rs_tree=0,rs_nt=0"),
]


@pytest.mark.parametrize("rows,n,dtype,op,knobs", SPLIT8_CASES, ids=lambda v: str(v))
def test_split_row_scan_of_8_byte_values(device, monkeypatch, rows, n, dtype, op, knobs):
    """In the interpreter's order, so bit for bit against the oracle."""
    if knobs:
        monkeypatch.setenv("CCHIP_TUNE", knobs)
    comb = {"add": D.add, "min": D.min, "max": D.max}[op]
    init = D.const(dtype, 0.5 if dtype is F64 else 3)
    g = Graph.create("split8", [("p", D.scan_rows(comb, init, D.param("x", dtype, (rows, n))))])
    lines = [l.split() for l in H.plan(g).splitlines() if l.startswith("kernel")]
    assert [(f[2], f[7]) for f in lines] == [("scan_rowseq", "320")], lines
    x = data(dtype, (rows, n), 131)
    exp = dict(oracle.run(g, [("x", x)]))["p"]
    c = H.compile(g)
    try:
        got = dict(H.run(c, [("x", x)]))["p"]
    finally:
        c.release()
    np.testing.assert_array_equal(got.view(np.uint8), exp.view(np.uint8))


SAME_FOLD_CASES = [
    # (shape, dtype, op, init, knobs, template): every scan template
    ((100, 37), I32, "add", 3, "", "scan_wave"),
    ((100, 50), F32, "add", 0.0, "", "scan_wave"),
    ((300, 1000), F32, "add", 0.0, "", "scan_tile"),
    ((200, 4097), F64, "add", 0.5, "", "scan_tile"),
    ((300, 1001), I64, "max", 3, "", "scan_tile_fold"),  # with a tree sibling
    ((5, 300001), I32, "add", 0, "", "scan_lookback"),
    ((8, 100003), F64, "add", 0.5, "", "scan_lookback"),
    ((1 << 18,), F32, "add", 0.0, "", "scan_lookback"),
    ((2048, 300), F32, "add", 0.0, "", "scan_rowseq"),
    ((1024, 40000), F32, "add", 0.0, "rs_tree=0", "scan_rowseq"),  # split roles
    ((1030, 5000), I64, "max", 3, "rs_tree=0,rs_nt=0", "scan_rowseq"),
    ((1100, 70), F64, "add", 0.5, "rs_depth=2", "scan_rowseq"),
]


@pytest.mark.parametrize("shape,dtype,op,iv,knobs,template", SAME_FOLD_CASES, ids=lambda v: str(v))
def test_same_fold_reduction_is_the_scans_row_end(device, monkeypatch, shape, dtype, op, iv, knobs, template):
    """A reduction with the scan's combine and init over the same tensor
    takes the scan's last element of every row, bit for bit; both against
    the oracle to the policy bar, and bit for bit where the scan folds in
    the interpreter's order or the combine is exact in any order."""
    if knobs:
        monkeypatch.setenv("CCHIP_TUNE", knobs)
    comb = {"add": D.add, "max": D.max}[op]
    init = D.const(dtype, iv)
    x = D.param("x", dtype, shape)
    one_d = len(shape) == 1
    outs = [("s", D.scan(comb, init, x) if one_d else D.scan_rows(comb, init, x)),
            ("r", D.reduce(comb, init, x) if one_d else D.reduce_rows(comb, init, x))]
    if template == "scan_tile_fold":
        outs.append(("m", D.reduce_rows(D.min, D.const(dtype, 0), x)))
    g = Graph.create("same_fold", outs)
    assert [t for t in templates(g) if t != "scan_init"] == [template]
    xv = data(dtype, shape, 97)
    exp = dict(oracle.run(g, [("x", xv)]))
    c = H.compile(g)
    try:
        got = dict(H.run(c, [("x", xv)]))
    finally:
        c.release()
    last = np.ascontiguousarray(got["s"][..., -1])
    np.testing.assert_array_equal(np.ascontiguousarray(got["r"]).reshape(last.shape).view(np.uint8),
                                  last.view(np.uint8))
    bad = [v for v in Diff.policy_check(g, list(exp.items()), list(got.items())) if not v.ok]
    assert not bad, bad
    if template == "scan_rowseq" or not dtype.is_float or op != "add":
        np.testing.assert_array_equal(got["r"].view(np.uint8), exp["r"].view(np.uint8))


ROWLAST_CASES = [
    # (rows, len, dtype, knobs): Monte Carlo's shape, ragged rows, long rows
    # folded in order with split roles, 8-byte values, two tiles in flight
    (1024, 64, I32, ""),
    (1500, 333, I32, ""),
    (2048, 9000, I32, "rs_tree=0"),
    (1030, 64, F64, ""),
    (4096, 64, F32, ""),
    (1100, 70, I32, "rs_depth=2"),
]


def row_last_graph(rows, n, dtype):
    """A row scan with a non-identity init; every row's last element
    gathered through a map over the scan and another tensor of the same
    shape, then output and summed: the Monte Carlo paths' final prices."""
    x = D.param("x", dtype, (rows, n))
    y = D.param("y", dtype, (rows, n))
    p = D.scan_rows(D.add, D.const(dtype, 5), x)
    m = D.map2(lambda a, b: D.add(D.mul(a, D.const(dtype, 3)), b), p, y)
    idx = D.map(lambda i: D.add(D.mul(i, D.const(I32, n)), D.const(I32, n - 1)), D.iota((rows,)))
    last = D.gather(idx, m)
    return Graph.create("rowlast", [("last", last), ("s", D.reduce(D.add, D.const(dtype, 0), last))])


@pytest.mark.parametrize("rows,n,dtype,knobs", ROWLAST_CASES, ids=lambda v: str(v))
def test_row_last_gather_reads_the_scans_side_buffer(device, monkeypatch, rows, n, dtype, knobs):
    """The gathered last elements come from the scan's side buffer: against
    the oracle (integers bit for bit), and bit for bit against the strided
    reads of the scan's output (rowlast=0)."""
    if knobs:
        monkeypatch.setenv("CCHIP_TUNE", knobs)
    g = row_last_graph(rows, n, dtype)
    assert "_last" in H.plan(g)
    ins = [("x", data(dtype, (rows, n), 71)), ("y", data(dtype, (rows, n), 72))]
    check(g, ins, ["scan_rowseq"])
    c = H.compile(g)
    try:
        got = dict(H.run(c, ins))
    finally:
        c.release()
    monkeypatch.setenv("CCHIP_TUNE", ",".join(k for k in (knobs, "rowlast=0") if k))
    assert "_last" not in H.plan(g)
    c = H.compile(g)
    try:
        ref = dict(H.run(c, ins))
    finally:
        c.release()
    np.testing.assert_array_equal(got["last"], ref["last"])


@pytest.mark.parametrize("dtype", [I32, F32])
def test_row_last_side_buffer_only_for_rows_as_long(device, dtype):
    """Two scans with side buffers (rows 100 and 50 long); the first
    gather's source adds the second scan reshaped to 100-long rows, which
    it must read in that scan's own buffer (at p * 100 + 99, the last
    element of its row 2p + 1), not in its side buffer at p."""
    from test_plan import _mixed_row_last_graph

    g = _mixed_row_last_graph(dtype)
    ins = [("x", data(dtype, (2048, 100), 74)), ("y", data(dtype, (4096, 50), 75))]
    check(g, ins, ["scan_rowseq"])


ROWLAST_MAP_CASES = [
    # (rows, len, dtype, knobs): the Greeks' paths tensor's shape; rows not
    # a multiple of the 4-element groups; a tail past the last group; 8-byte
    # groups of 2; two groups a lane (clamped last groups)
    (1024, 64, F32, ""),
    (1030, 70, I32, ""),
    (301, 7, I32, ""),
    (1000, 63, F64, ""),
    (1030, 66, I32, "map_unroll=2"),
]


def row_last_map_graph(rows, n, dtype):
    """A map materialised because two roots read it (the Greeks' paths);
    every row's last element gathered through another map, and output."""
    x = D.param("x", dtype, (rows, n))
    m = D.map(lambda v: D.add(D.mul(v, D.const(dtype, 2)), D.const(dtype, 1)), x)
    idx = D.map(lambda i: D.add(D.mul(i, D.const(I32, n)), D.const(I32, n - 1)), D.iota((rows,)))
    last = D.gather(idx, D.map(lambda v: D.mul(v, D.const(dtype, 3)), m))
    return Graph.create("rowlastm", [("last", last), ("t", D.reduce_rows(D.max, D.const(dtype, -100), m))])


@pytest.mark.parametrize("rows,n,dtype,knobs", ROWLAST_MAP_CASES, ids=lambda v: str(v))
def test_row_last_gather_reads_the_maps_side_buffer(device, monkeypatch, rows, n, dtype, knobs):
    """The same for a materialised map root: the map template stores each
    row's last element as it computes it."""
    if knobs:
        monkeypatch.setenv("CCHIP_TUNE", knobs)
    g = row_last_map_graph(rows, n, dtype)
    assert "_last" in H.plan(g)
    ins = [("x", data(dtype, (rows, n), 73))]
    check(g, ins, ["map"])
    c = H.compile(g)
    try:
        got = dict(H.run(c, ins))
    finally:
        c.release()
    monkeypatch.setenv("CCHIP_TUNE", ",".join(k for k in (knobs, "rowlast=0") if k))
    c = H.compile(g)
    try:
        ref = dict(H.run(c, ins))
    finally:
        c.release()
    np.testing.assert_array_equal(got["last"], ref["last"])


FOLDED_CASES = [((1 << 16) + 3, F32, "add"), ((1 << 22) + 5, F32, "add"), ((1 << 20) + 2, F64, "add"),
                (300 * 1024 + 5, F32, "add"), (1 << 18, F32, "add"), (102421, F32, "max"),
                ((1 << 22) + 1, I32, "add"), ((1 << 20) + 7, F32, "max"), (1 << 23, I32, "max"),
                ((1 << 21) + 1, F64, "max")]


@pytest.mark.parametrize("n,dtype,comb", FOLDED_CASES, ids=lambda v: str(v))
def test_reduce_folded_into_its_map(device, monkeypatch, n, dtype, comb):
    """A whole-tensor reduce of the previous root's map output folds inside
    the map kernel: one partial a wave (flagged where the wave held no
    element), then one fold kernel: up to 1024 partials in 256 threads, up
    to 16384 in one workgroup of 1024; past that, or past 1024 partials
    (2^18 4-byte elements) with fold_one=0, 1024 a workgroup and then a
    second kernel. Ragged tails, init not the identity (folded once),
    integers exact."""
    x, y = D.param("x", dtype, (n,)), D.param("y", dtype, (n,))
    r = D.map2(lambda a, b: D.add(D.mul(a, D.const(dtype, 2)), b), x, y)
    op = D.add if comb == "add" else D.max
    g = Graph.create("mr", [("r", r), ("s", D.reduce(op, D.const(dtype, 3), r))])
    t = templates(g)
    groups = n // (2 if dtype is F64 else 4)  # 16-byte groups, one a lane, 256 lanes a workgroup
    parts = 4 * -(-groups // 256)  # one partial a wave
    assert t[0] == "map" and "reduce_split" not in t, t
    assert t.count("reduce_split_fold") == (1 if parts <= 16384 else 2), (parts, t)
    ins = [("x", data(dtype, (n,), 31)), ("y", data(dtype, (n,), 32))]
    check(g, ins, ["map", "reduce_split_fold"])
    if 1024 < parts <= 16384:
        monkeypatch.setenv("CCHIP_TUNE", "fold_one=0")
        assert templates(g).count("reduce_split_fold") == 2
        check(g, ins, ["map", "reduce_split_fold"])


@pytest.mark.parametrize("order", ["sum_first", "map_first"])
def test_reduce_folded_with_fan_out(device, order):
    """A map output materialised only by its fan-out (two consumers, not an
    output): the sum folds inside the map kernel when it is the next root,
    and reads the output back when the other consumer's root comes
    between."""
    n = (1 << 20) + 3
    x, y = D.param("x", F32, (n,)), D.param("y", F32, (n,))
    r = D.map2(lambda a, b: D.add(D.mul(a, D.const(F32, 2)), b), x, y)
    s = D.reduce(D.add, D.const(F32, 0.5), r)
    q = D.map(lambda e: D.mul(e, e), r)
    outs = [("s", s), ("q", q)] if order == "sum_first" else [("q", q), ("s", s)]
    g = Graph.create("fan", outs)
    t = templates(g)
    assert ("reduce_split" in t) == (order == "map_first"), t
    check(g, [("x", data(F32, (n,), 33)), ("y", data(F32, (n,), 34))], ["map", "reduce_split_fold"])


def test_rows_max_min_tree_edges(device):
    """max and min of rows fold as a tree: IEEE maximum and minimum
    propagate NaN and order -0 below +0, so every row matches the
    interpreter's fold in order bit for bit (rows of zeros of both signs,
    infinities, NaNs); init applied once."""
    rows, n = 1024, 5000
    v = data(F32, (rows, n), 35)
    r = np.random.default_rng(5)
    v[r.integers(0, rows, 40), r.integers(0, n, 40)] = np.nan
    v[v > 0.999] = np.inf
    v[v < -0.999] = -np.inf
    v[100:110] = 0.0
    v[100:110, ::3] = -0.0
    v[200:210] = -0.0
    x = D.param("x", F32, (rows, n))
    g = Graph.create("mm", [("mx", D.reduce_rows(D.max, D.const(F32, -0.0), x)),
                            ("mn", D.reduce_rows(D.min, D.const(F32, 0.0), x))])
    assert templates(g) == ["reduce_block", "reduce_block"]
    exp = oracle.run(g, [("x", v)])
    c = H.compile(g)
    try:
        got = H.run(c, [("x", v)])
    finally:
        c.release()
    for (name, e), (_, d) in zip(exp, got):
        assert np.array_equal(np.isnan(e), np.isnan(d)), name
        ok = ~np.isnan(e)
        np.testing.assert_array_equal(e[ok].view(np.uint32), d[ok].view(np.uint32), err_msg=name)


def test_sibling_max_min_and_max_scan_edges(device):
    """The fused sibling kernel on the same edge values: row max and min
    and a max scan of rows of zeros of both signs, infinities and NaNs,
    bit for bit against the interpreter's in-order folds and scan."""
    rows, n = 1024, 5000
    v = data(F32, (rows, n), 36)
    r = np.random.default_rng(6)
    v[r.integers(0, rows, 40), r.integers(0, n, 40)] = np.nan
    v[v > 0.999] = np.inf
    v[v < -0.999] = -np.inf
    v[100:110] = 0.0
    v[100:110, ::3] = -0.0
    v[200:210] = -0.0
    x = D.param("x", F32, (rows, n))
    g = Graph.create("mm", [("mx", D.reduce_rows(D.max, D.const(F32, -0.0), x)),
                            ("q", D.scan_rows(D.max, D.const(F32, -0.0), x)),
                            ("mn", D.reduce_rows(D.min, D.const(F32, 0.0), x))])
    assert templates(g) == ["scan_tile_fold"]
    exp = oracle.run(g, [("x", v)])
    c = H.compile(g)
    try:
        got = H.run(c, [("x", v)])
    finally:
        c.release()
    for (name, e), (_, d) in zip(exp, got):
        assert np.array_equal(np.isnan(e), np.isnan(d)), name
        ok = ~np.isnan(e)
        np.testing.assert_array_equal(e[ok].view(np.uint32), d[ok].view(np.uint32), err_msg=name)


def test_reduce_empty_rows(device):
    x = D.param("x", F32, (5, 0))
    g = Graph.create("e", [("s", D.reduce_rows(D.add, D.const(F32, 2.5), x))])
    check(g, [("x", np.zeros((5, 0), np.float32))], ["reduce_empty"])


def test_scan_rows_exact_order_f32(device, monkeypatch):
    """With rs_tree=0 row scans, and with rr_tree=1 row sums, fold in the
    interpreter's order: bit-exact f32."""
    monkeypatch.setenv("CCHIP_TUNE", "rr_tree=1,rs_tree=0")
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


@pytest.mark.parametrize("n", [0, 1, 2, 3, 5, 1023, 1025, 65537])
@pytest.mark.parametrize("tune", ["", "map_nt=2"])
def test_map_ragged_8_byte(device, monkeypatch, n, tune):
    """Maps with an 8-byte operand take 2-element (16-byte) groups: f64 and
    i64 outputs, a mixed f32/f64 input pair, ragged tails, plain and
    streaming accesses."""
    if tune:
        monkeypatch.setenv("CCHIP_TUNE", tune)
    x = D.param("x", F64, (n,))
    y = D.param("y", F32, (n,))
    z = D.param("z", I64, (n,))
    g = Graph.create("m", [("r", D.map2(lambda a, b: D.add(D.mul(a, a), D.cast(F64, b)), x, y)),
                           ("f", D.map2(lambda a, b: D.mul(b, D.cast(F32, a)), x, y)),
                           ("q", D.map(lambda b: D.sub(D.mul(b, D.const(I64, 3)), D.const(I64, 1)), z))])
    check(g, [("x", data(F64, (n,), 3)), ("y", data(F32, (n,), 4)), ("z", data(I64, (n,), 5))],
          [] if n == 0 else ["map"])


def scatter_graph(n, bins, dtype):
    idx = D.param("idx", I32, (n,))
    src = D.param("src", dtype, (n,))
    return Graph.create("h", [("h", D.scatter_add(idx, src, (bins,)))])


def scatter_idx(seed, n, bins):
    v = C.philox_w0(seed, n).astype(np.int64) % bins
    if n >= 2:
        v[0], v[-1] = 0, bins - 1
    return v.astype(np.int32)


SCATTER_CASES = [
    # (n, bins, dtype, templates): one slice folded directly (with and
    # without partials), partitioned slices (with partials, and W = 1 where
    # each slice's table is stored straight to the output)
    (100003, 1000, F32, ["scatter_direct", "scatter_reduce"]),
    (100003, 1000, F64, ["scatter_direct", "scatter_reduce"]),
    (100003, 1000, I32, ["scatter_direct", "scatter_reduce"]),
    (5000, 4096, I32, ["scatter_direct"]),
    (300001, 50000, F32, ["scatter_partition", "scatter_accumulate", "scatter_reduce"]),
    (300001, 50000, F64, ["scatter_partition", "scatter_accumulate", "scatter_reduce"]),
    (300001, 50001, I32, ["scatter_partition", "scatter_accumulate", "scatter_reduce"]),
    # tile-local runs up to 256 slices, per-chunk offsets above
    ((1 << 20) + 3, 256 * 16384, F32, ["scatter_partition", "scatter_accumulate", "scatter_reduce"]),
    ((1 << 20) + 3, 256 * 16384 + 1, F32, ["scatter_count", "scatter_partition", "scatter_accumulate"]),
    ((1 << 20) + 3, 256 * 8192 + 1, F64, ["scatter_count", "scatter_partition", "scatter_accumulate"]),
    (1 << 20, (1 << 24) + 5, F32, ["scatter_partition", "scatter_accumulate"]),
    (1 << 20, 1 << 24, I32, ["scatter_partition", "scatter_accumulate"]),
]


@pytest.mark.parametrize("n,bins,dtype,tpl", SCATTER_CASES, ids=lambda v: str(v))
def test_scatter_paths(device, n, bins, dtype, tpl):
    g = scatter_graph(n, bins, dtype)
    if "scatter_reduce" not in tpl:
        assert "scatter_reduce" not in templates(g)
    check(g, [("idx", scatter_idx(3, n, bins)), ("src", data(dtype, (n,), 4))], tpl)


@pytest.mark.parametrize("dtype,tune", [(I32, ""), (F32, ""), (I32, "scatter_two_level=0"), (F64, "")])
def test_scatter_permutation_two_level(device, dtype, tune, monkeypatch):
    """Collision-free indices over more than 512 slices: a coarse pass into
    super-slices, then the slice pass (or, with scatter_two_level=0, one
    pass with element-wise stores)."""
    monkeypatch.setenv("CCHIP_TUNE", tune)
    n, bins = 1 << 22, 1 << (23 if dtype is F64 else 24)
    g = scatter_graph(n, bins, dtype)
    t = templates(g)
    assert ("scatter_coarse" in t) == (tune == "")
    idx = (C.permutation(31, bins)[:n]).astype(np.int32)
    check(g, [("idx", idx), ("src", data(dtype, (n,), 32))], ["scatter_partition", "scatter_accumulate"])


GATHER_BACK_CASES = [
    # (n, bins, dtype, two levels)
    ((1 << 20) + 37, 1 << 16, F32, False),
    (300001, 100003, I32, False),
    ((1 << 19) + 5, 1 << 17, F64, False),
    ((1 << 22) + 3, 1 << 24, F32, True),
    ((1 << 21) + 11, (1 << 24) + 1, I32, True),
    ((1 << 20) + 1, 1 << 23, F64, True),
    # three tiles a chunk, the last chunk one short tile (the partition marks
    # the tiles past the end empty)
    ((1 << 24) + 5, 1 << 20, F32, False),
    # 301 slices: one level, per-chunk offsets (no tile-local runs)
    ((1 << 21) + 7, 301 * 16384 - 5, F32, False),
    # 5001 slices in 79 super-slices (more than 64: two windows-table
    # entries a lane)
    ((1 << 20) + 5, 5000 * 16384 + 3, F32, True),
]


@pytest.mark.parametrize("n,bins,dtype,two", GATHER_BACK_CASES)
def test_gather_back_through_the_partition(device, n, bins, dtype, two, monkeypatch):
    """gather(idx, h) over h = scatter_add(idx, src, bins) reads h back
    through the scatter's partition (one level, or two above 512 slices):
    back is exactly h[idx], bit for bit, on ragged sizes and every dtype; h
    and back against the oracle under the policy; the same outputs as with
    the plain gather (scatter_gather_back=0), integers bit for bit."""
    g = C.scatter_gather(n, bins, dtype)
    t = templates(g)
    # the slice step is its own kernel, or (one workgroup a slice) part of
    # the accumulate
    back = t[t.index("scatter_accumulate") + 1:]
    assert back in (["gather_unpartition"] * (2 if two else 1),
                    ["scatter_reduce", "gather_slices"] + ["gather_unpartition"] * (2 if two else 1),
                    ["gather_slices"] + ["gather_unpartition"] * (2 if two else 1)), t
    assert ("scatter_coarse" in t) == two
    if two:
        idx = C.permutation(31, bins)[:n].astype(np.int32)
        idx[::7] = idx[3]  # and one crowded bin
    else:
        idx = scatter_idx(7, n, bins)
    inputs = [("idx", idx), ("src", data(dtype, (n,), 8))]
    check(g, inputs, ["gather_unpartition"])
    c = H.compile(g)
    try:
        o = dict(H.run(c, inputs))
    finally:
        c.release()
    np.testing.assert_array_equal(o["back"], o["h"][idx])
    monkeypatch.setenv("CCHIP_TUNE", "scatter_gather_back=0")
    assert templates(g)[-1] == "map"
    c = H.compile(g)
    try:
        plain = dict(H.run(c, inputs))
    finally:
        c.release()
    np.testing.assert_array_equal(plain["back"], plain["h"][idx])
    if dtype is I32:
        np.testing.assert_array_equal(o["h"], plain["h"])
        np.testing.assert_array_equal(o["back"], plain["back"])


@pytest.mark.parametrize("bad", [1, -1, None])
def test_one_element_gather(device, bad):
    """A gather from a one-element tensor (how a gradient spreads a whole
    sum's adjoint) reads that element at any index in range, loaded once
    outside the kernel's loop; an index out of range still raises, and a
    good run after it is clean."""
    n = 70001
    x, idx = D.param("x", F32, (n,)), D.param("idx", I32, (n,))
    tot = D.reduce(D.add, D.const(F32, 0.0), x)
    g = Graph.create("g1", [("o", D.map2(D.mul, x, D.gather(idx, D.map(lambda v: D.mul(v, v), tot))))])
    xv = data(F32, (n,), 41)
    iv = np.zeros(n, np.int32)
    c = H.compile(g)
    try:
        if bad is not None:
            biv = iv.copy()
            biv[n - 1] = bad
            with pytest.raises(ValueError, match="gather index out of bounds"):
                H.run(c, [("x", xv), ("idx", biv)])
        got = dict(H.run(c, [("x", xv), ("idx", iv)]))["o"]
    finally:
        c.release()
    exp = dict(oracle.run(g, [("x", xv), ("idx", iv)]))["o"]
    bad_v = [v for v in Diff.policy_check(g, [("o", exp)], [("o", got)]) if not v.ok]
    assert not bad_v, bad_v


@pytest.mark.parametrize("two", [False, True])
def test_gather_back_out_of_range_raises(device, two):
    """An index out of range is skipped by the scatter's partition, so it
    has no slot: the run raises the gather's error, and the next run with
    good indices is clean."""
    n, bins = (1 << 20) + 3, (1 << 22 if two else 1 << 16)
    g = C.scatter_gather(n, bins, F32)
    idx = scatter_idx(9, n, bins)
    bad = idx.copy()
    bad[n // 2] = bins + 5
    bad[7] = -1
    src = data(F32, (n,), 10)
    c = H.compile(g)
    try:
        with pytest.raises(ValueError, match="gather index out of bounds"):
            H.run(c, [("idx", bad), ("src", src)])
        o = dict(H.run(c, [("idx", idx), ("src", src)]))
        np.testing.assert_array_equal(o["back"], o["h"][idx])
    finally:
        c.release()


@pytest.mark.parametrize("dtype", [F32, I32])
def test_scatter_atomic_path(device, dtype, monkeypatch):
    """The global-atomic template, still used where the slices would not
    fit (and selectable with scatter_lds=0)."""
    monkeypatch.setenv("CCHIP_TUNE", "scatter_lds=0")
    n, bins = 100003, 50000
    check(scatter_graph(n, bins, dtype), [("idx", scatter_idx(5, n, bins)), ("src", data(dtype, (n,), 6))],
          ["scatter_zero", "scatter_atomic"])


@pytest.mark.parametrize("dtype", [F32, F64, I32])
def test_broadcast_read_from_its_source(device, dtype):
    """Broadcasts the fusion plan materialises, read by their consumers
    from the one-element source (the broadcast's own kernel dropped), with
    a broadcast output and a matrix-core operand that keep theirs; against
    the oracle."""
    s = D.scalar("s", dtype)
    x = D.param("x", dtype, (300, 257))
    b = D.broadcast((300, 257), s)
    g = Graph.create("bc", [("u", D.map2(D.add, b, x)), ("v", D.map2(D.mul, b, x)),
                            ("r", D.reduce_rows(D.add, D.const(dtype, 0), D.map2(D.sub, x, b))),
                            ("p", D.scan_rows(D.max, D.const(dtype, -100), D.map2(D.add, b, x)))])
    assert "elided" in H.plan(g)
    sv = np.array(3, np.int32) if dtype is I32 else np.array(0.375, dtype.np)
    check(g, [("s", sv), ("x", data(dtype, (300, 257), 24))], [])
    # a map of the broadcast, materialised and computed by its consumers
    e = D.map(lambda v: D.mul(D.add(v, D.const(dtype, 1)), v), b)
    g2 = Graph.create("bc2", [("u", D.map2(D.add, e, x)), ("v", D.map2(D.sub, x, e))])
    assert H.plan(g2).count("elided") == 1
    check(g2, [("s", sv), ("x", data(dtype, (300, 257), 26))], [])
    if dtype is not I32:
        b2, x2 = D.broadcast((256, 256), s), D.param("x", dtype, (256, 256))
        g3 = Graph.create("bc3", [("c", D.matmul(b2, x2)), ("v", D.map2(D.mul, b2, x2)), ("b", b2)])
        check(g3, [("s", sv), ("x", data(dtype, (256, 256), 25))], [])


@pytest.mark.parametrize("dtype", [F32, F64, I32])
def test_affine_scatter_read_in_place(device, dtype):
    """A scatter_add through an injective affine index in range, read by a
    map at its own index, gathered at random indices, reduced and scanned
    by max, and read as a matmul operand, each computing its elements in
    place (no scatter kernel): bit-exact against the oracle, including a
    -0.0 source landing as +0.0 and NaN/inf sources."""
    n = 100003
    for a, b, m in [(3, 1, 3 * n + 5), (-2, 2 * n + 7, 2 * n + 9), (64, 63, 64 * n)]:
        idx = D.map(lambda p: D.add(D.mul(p, D.const(I32, a)), D.const(I32, b)), D.iota((n,)))
        src, y = D.param("src", dtype, (n,)), D.param("y", dtype, (m,))
        gi = D.param("gi", I32, (5000,))
        h = D.scatter_add(idx, D.map(lambda v: D.add(v, v), src), (m,))
        one = D.const(dtype, 1 if not dtype.is_float else 1.0)
        g1 = Graph.create("inplace", [("o", D.map2(lambda u, v: D.add(D.mul(u, v), u), h, y)),
                                      ("g", D.gather(gi, h))])
        lo = D.const(dtype, -(1 << 30) if not dtype.is_float else -1e30)
        g2 = Graph.create("inplace2", [("mx", D.reduce(D.max, lo, D.map(lambda u: D.add(u, one), h))),
                                       ("sc", D.scan(D.max, lo, h))])
        for g in (g1, g2):
            assert "scatter_affine" not in templates(g), (a, b, templates(g))
        x = data(dtype, (n,), 31)
        ins = [("src", x), ("y", data(dtype, (m,), 32)),
               ("gi", np.random.default_rng(33).integers(0, m, size=5000).astype(np.int32))]
        for g, special in ((g1, True), (g2, False)):
            xs = x.copy()
            if special and dtype.is_float:
                xs[:8] = [-0.0, np.nan, np.inf, -np.inf, 0.0, -1.5, 2.5, -0.0]
            gins = [(k, xs if k == "src" else v) for k, v in ins if k in {nm for nm, _ in g.params}]
            exp = dict(oracle.run(g, gins))
            c = H.compile(g)
            try:
                got = dict(H.run(c, gins))
            finally:
                c.release()
            for k in exp:
                np.testing.assert_array_equal(np.atleast_1d(got[k]).view(np.uint8), np.atleast_1d(exp[k]).view(np.uint8),
                                              err_msg="%s %s %s" % (a, b, k))
    if dtype in (F32, F64):
        # a matmul operand computes it as its element function
        src = D.param("src", dtype, (1 << 14,))
        idx = D.map(lambda p: D.add(D.mul(p, D.const(I32, 64)), D.const(I32, 63)), D.iota((1 << 14,)))
        h = D.scatter_add(idx, src, (1 << 20,))
        g = Graph.create("mm", [("c", D.matmul(D.reshape((1024, 1024), h), D.param("w", dtype, (1024, 64))))])
        assert "scatter_affine" not in templates(g)
        check(g, [("src", data(dtype, (1 << 14,), 34)), ("w", data(dtype, (1024, 64), 35))], [])


@pytest.mark.parametrize("dtype", [F32, F64, I32])
def test_scatter_affine_index(device, dtype):
    """scatter_add through an index a*i + b built from iota (a strided,
    reversed, offset index; also through a reshape): one pass over the bins,
    bit-exact against the oracle, including each hit bin's 0 + x (a -0.0
    source lands as +0.0) and NaN/inf sources; an affine index that leaves
    the range takes the general path and raises."""
    n = 300007
    for a, b, m in [(3, 1, 3 * n + 5), (-2, 2 * n + 7, 2 * n + 9), (1, 0, n), (64, 63, 64 * n)]:
        idx = D.map(lambda p: D.add(D.mul(p, D.const(I32, a)), D.const(I32, b)), D.iota((n,)))
        src = D.param("src", dtype, (n,))
        g = Graph.create("aff", [("h", D.scatter_add(idx, src, (m,)))])
        assert templates(g) == ["scatter_affine"], (a, b, templates(g))
        x = data(dtype, (n,), 21)
        if dtype is not I32:
            x[:8] = [-0.0, np.nan, np.inf, -np.inf, 0.0, -1.5, 2.5, -0.0]
        exp = oracle.run(g, [("src", x)])
        c = H.compile(g)
        try:
            got = H.run(c, [("src", x)])
        finally:
            c.release()
        np.testing.assert_array_equal(got[0][1].view(np.uint8), exp[0][1].view(np.uint8))
    # through a reshape of a 2-d iota
    idx = D.reshape((7007,), D.map(lambda p: D.sub(D.mul(p, D.const(I32, 2)), D.const(I32, -5)), D.iota((7, 1001))))
    g = Graph.create("aff2", [("h", D.scatter_add(idx, D.param("src", dtype, (7007,)), (2 * 7007 + 5,)))])
    assert templates(g) == ["scatter_affine"]
    check(g, [("src", data(dtype, (7007,), 22))], ["scatter_affine"])
    # out of range: the general path, which raises
    idx = D.map(lambda p: D.mul(p, D.const(I32, 2)), D.iota((1000,)))
    g = Graph.create("aff3", [("h", D.scatter_add(idx, D.param("src", dtype, (1000,)), (1500,)))])
    assert "scatter_affine" not in templates(g)
    c = H.compile(g)
    try:
        with pytest.raises(ValueError, match="scatter_add index out of bounds"):
            H.run(c, [("src", data(dtype, (1000,), 23))])
    finally:
        c.release()


def test_scatter_two_level_empty_super_slices(device):
    """Two levels with most super-slices empty and two crowded ones: the
    slice pass's windows all fall in those two (one of them over many
    windows), with a gather back."""
    n, bins = (1 << 20) + 9, 1 << 24
    r = np.random.default_rng(5)
    idx = np.where(r.random(n) < 0.8, r.integers(0, 1 << 18, n), r.integers(bins - 1024, bins, n)).astype(np.int32)
    g = C.scatter_gather(n, bins, F32)
    assert "scatter_coarse" in templates(g)
    inputs = [("idx", idx), ("src", data(F32, (n,), 9))]
    check(g, inputs, ["gather_unpartition"])
    c = H.compile(g)
    try:
        o = dict(H.run(c, inputs))
    finally:
        c.release()
    np.testing.assert_array_equal(o["back"], o["h"][idx])


@pytest.mark.parametrize("bins", [3000, 70000])
def test_scatter_one_hot_bin(device, bins):
    """Every element in one bin: one slice takes all the work."""
    n = 200000
    idx = np.full(n, bins // 2, np.int32)
    check(scatter_graph(n, bins, I32), [("idx", idx), ("src", data(I32, (n,), 7))], [])
    check(scatter_graph(n, bins, F32), [("idx", idx), ("src", data(F32, (n,), 8))], [])


def test_scatter_empty_source(device):
    check(scatter_graph(0, 10, F32), [("idx", np.zeros(0, np.int32)), ("src", np.zeros(0, np.float32))],
          ["scatter_zero"])


def test_scatter_fused_operands(device):
    """Index and source are fused expressions, evaluated in both the count
    and the partition pass."""
    n, bins = 200000, 30000
    i = D.param("i", I32, (n,))
    x = D.param("x", F32, (n,))
    idx = D.map(lambda e: D.sub(D.const(I32, bins - 1), D.mul(e, D.const(I32, 1))), i)
    g = Graph.create("h", [("h", D.scatter_add(idx, D.map(D.exp, x), (bins,)))])
    check(g, [("i", scatter_idx(9, n, bins)), ("x", data(F32, (n,), 10))], ["scatter_partition"])


@pytest.mark.parametrize("bins", [4, 50000, 1 << 23])
def test_scatter_partition_out_of_range_raises(device, bins):
    n = 20000
    idx = scatter_idx(11, n, bins)
    idx[777] = bins
    idx[12345] = -1
    c = H.compile(scatter_graph(n, bins, I32))
    try:
        with pytest.raises(ValueError, match="scatter_add index out of bounds"):
            H.run(c, [("idx", idx), ("src", np.ones(n, np.int32))])
        idx[777], idx[12345] = 0, 1
        got = dict(H.run(c, [("idx", idx), ("src", np.ones(n, np.int32))]))["h"]
        np.testing.assert_array_equal(got, np.bincount(idx, minlength=bins).astype(np.int32))
    finally:
        c.release()


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


KNOB_CASES = [
    # (knob setting, graph builder, inputs builder, template that must appear)
    ("lb_window=4", lambda: Graph.create("s", [("p", D.scan_rows(D.add, D.const(I32, 3), D.param("x", I32, (3, 300001))))]),
     lambda: [("x", data(I32, (3, 300001), 41))], "scan_lookback"),
    # long look-back scans use exact types: a tree-ordered f32 prefix sum of
    # this length and the interpreter's sequential one differ by more than
    # the 1e-4 band near zero, whichever is closer to the exact sum
    ("lb_window=2,lb_slices4=8", lambda: Graph.create("s", [("p", D.scan_rows(D.add, D.const(I32, 0), D.param("x", I32, (2, 200003))))]),
     lambda: [("x", data(I32, (2, 200003), 42))], "scan_lookback"),
    ("lb_slices8=4", lambda: Graph.create("s", [("p", D.scan_rows(D.add, D.const(I64, 0), D.param("x", I64, (2, 100003))))]),
     lambda: [("x", data(I64, (2, 100003), 56))], "scan_lookback"),
    ("mm_bk=32,mm_chunk_k=0", lambda: C.matmul(256, F32, k=512, m=128),
     lambda: [("a", data(F32, (128, 512), 43)), ("b", data(F32, (512, 256), 44))], "matmul_mfma_f32_a0b0"),
    ("mm_f64_bm=128,mm_f64_bk=32", lambda: C.matmul(256, F64, k=128, m=256),
     lambda: [("a", data(F64, (256, 128), 45)), ("b", data(F64, (128, 256), 46))], "matmul_mfma_f64_a0b0"),
    # the f64 kernel double-buffered without the register budget
    ("mm_f64_single=0,mm_f64_waves=0", lambda: C.matmul(192, F64, k=320, m=256),
     lambda: [("a", data(F64, (256, 320), 93)), ("b", data(F64, (320, 192), 94))], "matmul_mfma_f64_a0b0"),
    ("mm_f64_waves=6", lambda: C.matmul_grad(128, F64),
     lambda: [("a", data(F64, (128, 128), 95)), ("b", data(F64, (128, 128), 96))], "matmul_mfma_f64_a1b0"),
    ("mm_kpad=3,mm_mpad=2", lambda: C.matmul_grad(256, F32),
     lambda: [("a", data(F32, (256, 256), 47)), ("b", data(F32, (256, 256), 48))], "matmul_mfma_f32_a1b0"),
    # tile order inside each XCD's run of tile rows: column by column (the
    # default; a non-square grid of 16 x 8 tiles) and row by row
    ("mm_xcd_cols=1", lambda: C.matmul(1024, F32, k=64, m=2048),
     lambda: [("a", data(F32, (2048, 64), 51)), ("b", data(F32, (64, 1024), 52))], "matmul_mfma_f32_a0b0"),
    ("mm_xcd_cols=0", lambda: C.matmul(1024, F64, k=64, m=1024),
     lambda: [("a", data(F64, (1024, 64), 53)), ("b", data(F64, (64, 1024), 54))], "matmul_mfma_f64_a0b0"),
    ("mm_mfma=0", lambda: C.matmul(128, F32, k=64, m=128),
     lambda: [("a", data(F32, (128, 64), 49)), ("b", data(F32, (64, 128), 50))], "matmul_tiled"),
    ("map_nt=2", lambda: P.chain(5000).graph(), lambda: P.chain(5000).inputs(), "map"),
    ("scatter_slice_bins=8192", lambda: scatter_graph(300001, 70000, F32),
     lambda: [("idx", scatter_idx(51, 300001, 70000)), ("src", data(F32, (300001,), 52))], "scatter_partition"),
    ("rs_groups=512", lambda: C.rows(8192, 1000), lambda: [("x", data(F32, (8192, 1000), 77))], "scan_rowseq"),
    ("rs_tree=0,rs_bytes=8192,rs_groups=64", lambda: C.rows(1024, 3000),
     lambda: [("x", data(F32, (1024, 3000), 53))], "scan_rowseq"),
    ("mm_splitk_groups=7", lambda: C.matmul(3, F64, k=65536, m=3),
     lambda: [("a", data(F64, (3, 65536), 54)), ("b", data(F64, (65536, 3), 55))], "matmul_splitk"),
    # streaming (non-temporal) access masks, the default of each being 3 / 5
    ("scan_nt=0", lambda: Graph.create("s", [("p", D.scan_rows(D.add, D.const(I32, 1), D.param("x", I32, (2, 300004))))]),
     lambda: [("x", data(I32, (2, 300004), 57))], "scan_lookback"),
    ("scan_nt=1", lambda: Graph.create("s", [("p", D.scan_rows(D.add, D.const(I64, 0), D.param("x", I64, (1, 200000))))]),
     lambda: [("x", data(I64, (1, 200000), 58))], "scan_lookback"),
    ("rs_tree=0,rs_nt=0", lambda: C.rows(1024, 3000), lambda: [("x", data(F32, (1024, 3000), 59))], "scan_rowseq"),
    ("rs_nt=2", lambda: C.rows(2048, 1000), lambda: [("x", data(F32, (2048, 1000), 60))], "reduce_rowseq"),
    ("rr_tree=1,rr_bytes=16384,rr_groups=64,same_fold=0", lambda: C.rows(1500, 2001),
     lambda: [("x", data(F32, (1500, 2001), 61))], "reduce_rowseq"),
    # two tiles in flight: an odd tile count with a ragged last tile
    ("rs_tree=0,rs_depth=2,rs_bytes=4096,rr_depth=2,rr_bytes=16384", lambda: C.rows(1024, 3000),
     lambda: [("x", data(F32, (1024, 3000), 62))], "scan_rowseq"),
    ("rs_tree=0,rr_tree=1,rr_depth=2,rr_bytes=16384,same_fold=0", lambda: C.rows(2048, 5003),
     lambda: [("x", data(F32, (2048, 5003), 63))], "reduce_rowseq"),
    ("rs_tree=0,rs_chunk=4,rr_chunk=128", lambda: C.rows(1024, 3000), lambda: [("x", data(F32, (1024, 3000), 64))], "scan_rowseq"),
    # long rows folded in order: floats bit-identical to the interpreter,
    # integers too (rows of four tiles or more, split roles, and a last
    # workgroup past the rows); rows just below and at the tree's length
    ("rr_tree=1", lambda: Graph.create("r", [("s", D.reduce_rows(D.add, D.const(F32, 0.5), D.param("x", F32, (1024, 20003))))]),
     lambda: [("x", data(F32, (1024, 20003), 60))], "reduce_rowseq"),
    ("rr_tree_len=2048", lambda: Graph.create("r", [("s", D.reduce_rows(D.max, D.const(I32, 3), D.param("x", I32, (1500, 2047))))]),
     lambda: [("x", data(I32, (1500, 2047), 63))], "reduce_rowseq"),
    # the tile scans' row length, both ways
    ("rs_tree_len=4096", lambda: Graph.create("s", [("p", D.scan_rows(D.max, D.const(I32, -7), D.param("x", I32, (1100, 3000))))]),
     lambda: [("x", data(I32, (1100, 3000), 65))], "scan_rowseq"),
    ("rs_tree_len=512", lambda: Graph.create("s", [("p", D.scan_rows(D.add, D.const(I32, 2), D.param("x", I32, (1030, 1000))))]),
     lambda: [("x", data(I32, (1030, 1000), 66))], "scan_tile"),
    ("rr_tree_len=64", lambda: Graph.create("r", [("s", D.reduce_rows(D.add, D.const(F32, 1.0), D.param("x", F32, (2000, 64))))]),
     lambda: [("x", data(F32, (2000, 64), 64))], "reduce_wave"),
    ("rr_tree=0", lambda: Graph.create("r", [("s", D.reduce_rows(D.add, D.const(I32, 5), D.param("x", I32, (1030, 30000))))]),
     lambda: [("x", data(I32, (1030, 30000), 61))], "reduce_rowseq"),
    ("rr_tree=0,rr_split=1", lambda: Graph.create("r", [("m", D.reduce_rows(D.max, D.const(I32, 3), D.param("x", I32, (1030, 30000))))]),
     lambda: [("x", data(I32, (1030, 30000), 62))], "reduce_rowseq"),
    # one workgroup folding and loading in turn for the scan, split roles for
    # the reductions (the defaults the other way round), and split f64 ones
    ("rs_tree=0,rs_split=0,rr_split=1", lambda: C.rows(1024, 20003), lambda: [("x", data(F32, (1024, 20003), 98))], "scan_rowseq"),
    ("rr_tree=1,rr_split=1", lambda: (lambda x: Graph.create("r", [("s", D.reduce_rows(D.add, D.const(F64, 1.5), x)),
                                                        ("m", D.reduce_rows(D.max, D.const(F64, 0.25), x))]))(
        D.param("x", F64, (4096, 5000))),
     lambda: [("x", data(F64, (4096, 5000), 99))], "reduce_rowseq"),
    # tiles of a non-power-of-two width (384 and 1536 columns)
    ("rs_tree=0,rs_bytes=6144,rr_bytes=24576", lambda: C.rows(1024, 3000),
     lambda: [("x", data(F32, (1024, 3000), 96))], "scan_rowseq"),
    ("lb_buf=0", lambda: Graph.create("s", [("p", D.scan_rows(D.add, D.const(I32, 2), D.param("x", I32, (3, 100001))))]),
     lambda: [("x", data(I32, (3, 100001), 65))], "scan_lookback"),
    ("scatter_prefetch=0", lambda: scatter_graph(300001, 70000, F32),
     lambda: [("idx", scatter_idx(68, 300001, 70000)), ("src", data(F32, (300001,), 69))], "scatter_partition"),
    # fewer, longer partition chunks: three and five tiles a workgroup, the
    # last one ragged, with gather back
    ("scatter_chunks=16", lambda: C.scatter_gather(300001, 70000, F32),
     lambda: [("idx", scatter_idx(91, 300001, 70000)), ("src", data(F32, (300001,), 92))], "gather_unpartition"),
    ("scatter_chunks=256", lambda: C.scatter_gather((1 << 23) + 5, 1 << 20, F32),
     lambda: [("idx", scatter_idx(93, (1 << 23) + 5, 1 << 20)), ("src", data(F32, ((1 << 23) + 5,), 94))],
     "gather_unpartition"),
    # threads per workgroup of the partition, accumulate and gather-back
    # kernels, away from their defaults (1024; 1024, or 512 with one
    # workgroup a slice; 512), with gather back
    ("scatter_part_threads=256,scatter_acc_threads=256,gather_threads=256",
     lambda: C.scatter_gather(300001, 70000, F32),
     lambda: [("idx", scatter_idx(81, 300001, 70000)), ("src", data(F32, (300001,), 82))], "gather_unpartition"),
    # the slice pass of two levels over counted chunks instead of windows
    ("scatter_windows=0", lambda: C.scatter_gather((1 << 21) + 11, (1 << 24) + 1, F32),
     lambda: [("idx", scatter_idx(87, (1 << 21) + 11, (1 << 24) + 1)), ("src", data(F32, ((1 << 21) + 11,), 88))],
     "scatter_coarse"),
    # the gather's slice step as its own kernel where one workgroup a slice
    # could have done it (one level with counted chunks; two levels)
    ("scatter_fuse_back=0", lambda: C.scatter_gather((1 << 21) + 7, 301 * 16384 - 5, F32),
     lambda: [("idx", scatter_idx(89, (1 << 21) + 7, 301 * 16384 - 5)), ("src", data(F32, ((1 << 21) + 7,), 90))],
     "gather_slices"),
    ("scatter_fuse_back=0", lambda: C.scatter_gather((1 << 21) + 11, (1 << 24) + 1, I32),
     lambda: [("idx", scatter_idx(91, (1 << 21) + 11, (1 << 24) + 1)), ("src", data(I32, ((1 << 21) + 11,), 92))],
     "gather_slices"),
    # per-chunk offsets instead of tile-local runs, with gather back
    ("scatter_local_max=0", lambda: C.scatter_gather((1 << 20) + 37, 1 << 16, F32),
     lambda: [("idx", scatter_idx(85, (1 << 20) + 37, 1 << 16)), ("src", data(F32, ((1 << 20) + 37,), 86))],
     "scatter_count"),
    ("scatter_part_threads=512,scatter_acc_threads=1024,gather_threads=1024",
     lambda: C.scatter_gather((1 << 20) + 1, 1 << 22, F64),
     lambda: [("idx", scatter_idx(83, (1 << 20) + 1, 1 << 22)), ("src", data(F64, ((1 << 20) + 1,), 84))],
     "gather_unpartition"),
    # the look-back's own fold of a predecessor tile that has not published
    # (taken after lb_spin polls; one poll forces it on nearly every wait):
    # row-start tiles with a non-identity init, floats, many small tiles
    ("lb_spin=1", lambda: Graph.create("s", [("p", D.scan_rows(D.add, D.const(I32, 2), D.param("x", I32, (3, 100001))))]),
     lambda: [("x", data(I32, (3, 100001), 70))], "scan_lookback"),
    ("lb_spin=1,lb_slices4=2", lambda: Graph.create("s", [("p", D.scan(D.add, D.const(I32, 0), D.param("x", I32, (50001,))))]),
     lambda: [("x", data(I32, (50001,), 71))], "scan_lookback"),
    ("lb_spin=1", lambda: Graph.create("s", [("p", D.scan_rows(D.add, D.const(F32, 0.5), D.param("x", F32, (2, 200000))))]),
     lambda: [("x", np.abs(data(F32, (2, 200000), 72)))], "scan_lookback"),
    ("lb_spin=1,lb_window=4", lambda: Graph.create("s", [("p", D.scan_rows(D.max, D.const(I32, -5), D.param("x", I32, (2, 300004))))]),
     lambda: [("x", data(I32, (2, 300004), 73))], "scan_lookback"),
    # four-wave look-back tiles (the default is eight)
    ("lb_waves=4", lambda: Graph.create("s", [("p", D.scan_rows(D.add, D.const(I32, 2), D.param("x", I32, (3, 300001))))]),
     lambda: [("x", data(I32, (3, 300001), 78))], "scan_lookback"),
    ("lb_waves=4,lb_spin=1", lambda: Graph.create("s", [("p", D.scan_rows(D.add, D.const(I32, 1), D.param("x", I32, (2, 200003))))]),
     lambda: [("x", data(I32, (2, 200003), 79))], "scan_lookback"),
    # float prefix sums of positive values, so that no prefix sits near a
    # zero crossing, where any summation order other than the oracle's
    # sequential one can leave the 1e-4 band
    ("lb_waves=4,lb_spin=1", lambda: Graph.create("s", [("p", D.scan_rows(D.add, D.const(F32, 0.5), D.param("x", F32, (2, 200003))))]),
     lambda: [("x", np.abs(data(F32, (2, 200003), 79)))], "scan_lookback"),
    ("lb_waves=4", lambda: Graph.create("s", [("p", D.scan_rows(D.add, D.const(I64, 0), D.param("x", I64, (1, 200000))))]),
     lambda: [("x", data(I64, (1, 200000), 80))], "scan_lookback"),
    # tiles from the atomic counter instead of blockIdx
    ("lb_counter=1", lambda: Graph.create("s", [("p", D.scan_rows(D.add, D.const(I32, 1), D.param("x", I32, (2, 300004))))]),
     lambda: [("x", data(I32, (2, 300004), 74))], "scan_lookback"),
    # groups per lane in the map template: a light map forced to two and three
    # (ragged tails, clamped last groups), a heavy one forced back to one
    ("map_unroll=2", lambda: P.chain(5003).graph(), lambda: P.chain(5003).inputs(), "map"),
    ("map_unroll=3", lambda: RB.poly_graph(10001, F64), lambda: [("x", RB.x_input(10001, F64))], "map"),
    ("map_unroll=1", lambda: RB.poly_graph(70001, F64), lambda: [("x", RB.x_input(70001, F64))], "map"),
    # a capped grid: lanes loop over several workgroup-wide runs
    ("map_blocks=3", lambda: P.chain(300007).graph(), lambda: P.chain(300007).inputs(), "map"),
    ("map_blocks=5,map_unroll=2", lambda: RB.poly_graph(100003, F64), lambda: [("x", RB.x_input(100003, F64))], "map"),
    ("map_blocks=7", lambda: Graph.create("aff", [("h", D.scatter_add(
        D.map(lambda p: D.add(D.mul(p, D.const(I32, 3)), D.const(I32, 1)), D.iota((100003,))),
        D.param("src", F32, (100003,)), (300014,)))]),
     lambda: [("src", data(F32, (100003,), 81))], "scatter_affine"),
    # 8-byte row scans storing 4-element groups instead of pairs
    ("rs_pairs8=0", lambda: Graph.create("s", [("p", D.scan_rows(D.add, D.const(F64, 1.0), D.param("x", F64, (1030, 68))))]),
     lambda: [("x", data(F64, (1030, 68), 82))], "scan_rowseq"),
    ("rs_pairs8=1,rs_nt=1", lambda: Graph.create("s", [("p", D.scan_rows(D.add, D.const(I64, 3), D.param("x", I64, (1100, 36))))]),
     lambda: [("x", data(I64, (1100, 36), 83))], "scan_rowseq"),
    # one-tile-a-row scans with every streaming mask
    ("rt_nt=3", lambda: Graph.create("s", [("p", D.scan_rows(D.max, D.const(I32, -7), D.param("x", I32, (300, 5001))))]),
     lambda: [("x", data(I32, (300, 5001), 84))], "scan_tile"),
    ("rt_nt=2", lambda: sibling_graph(I32, 600, 3001), lambda: [("x", data(I32, (600, 3001), 85))], "scan_tile_fold"),
    ("rt_nt=0", lambda: sibling_graph(I32, 600, 3000), lambda: [("x", data(I32, (600, 3000), 86))], "scan_tile_fold"),
    # the scatter chain's streaming and walk depths (tile-local partition;
    # two levels with windows)
    ("sp_nt=3,acc_nt=1,gs_nt=3,gb_nt=0", lambda: C.scatter_gather(200003, 1 << 18, I32),
     lambda: [("idx", scatter_idx(87, 200003, 1 << 18)), ("src", data(I32, (200003,), 88))], "gather_unpartition"),
    ("acc_groups=4,gb_groups=3", lambda: C.scatter_gather(200003, 1 << 18, I32),
     lambda: [("idx", scatter_idx(89, 200003, 1 << 18)), ("src", data(I32, (200003,), 90))], "scatter_accumulate"),
    ("gb_nt=3,gs_nt=2,acc_groups=3", lambda: C.scatter_gather(300001, 1 << 24, I32),
     lambda: [("idx", scatter_idx(91, 300001, 1 << 24)), ("src", data(I32, (300001,), 92))], "scatter_windows"),
    # the final prices read through the strided gather again
    ("rowlast=0", lambda: C.mc_paths(2048, 64), lambda: bs.inputs(F32, seed=7), "scan_rowseq"),
    # the map's loads and stores streamed each on its own
    ("map_ntl=0,map_nts=1", lambda: P.chain(300007).graph(), lambda: P.chain(300007).inputs(), "map"),
    ("map_ntl=1,map_nts=0", lambda: P.chain(300007).graph(), lambda: P.chain(300007).inputs(), "map"),
    # every streaming default taken as if the tensors were large
    ("nt_bytes=0", lambda: C.rows(2048, 1000), lambda: [("x", data(F32, (2048, 1000), 101))], "scan_rowseq"),
    ("nt_bytes=0", lambda: C.scatter_gather(200003, 1 << 18, F32),
     lambda: [("idx", scatter_idx(102, 200003, 1 << 18)), ("src", data(F32, (200003,), 103))], "gather_unpartition"),
    ("red_nt=1", lambda: Graph.create("r", [("s", D.reduce(D.add, D.const(F32, 0.5), D.param("x", F32, (300001,))))]),
     lambda: [("x", data(F32, (300001,), 104))], "reduce_split"),
    ("red_nt=1", lambda: Graph.create("r", [("m", D.reduce_rows(D.max, D.const(F32, 0), D.param("x", F32, (64, 30001))))]),
     lambda: [("x", data(F32, (64, 30001), 105))], "reduce_split"),
    # the counted partition's bucket counters in one and two copies
    ("scatter_local_max=0,scatter_count_copies=1", lambda: C.scatter_gather((1 << 20) + 37, 1 << 16, F32),
     lambda: [("idx", scatter_idx(106, (1 << 20) + 37, 1 << 16)), ("src", data(F32, ((1 << 20) + 37,), 107))],
     "scatter_count"),
    ("scatter_local_max=0,scatter_count_copies=2", lambda: scatter_graph(300001, 70000, I32),
     lambda: [("idx", scatter_idx(108, 300001, 70000)), ("src", data(I32, (300001,), 109))], "scatter_count"),
    # shapes: the one-slice fold over three workgroups, 128 KiB slice
    # tables, few accumulate workgroups, two levels from eight slices up,
    # 4096-element partition tiles
    ("scatter_direct_wgs=3", lambda: scatter_graph(300001, 5000, F32),
     lambda: [("idx", scatter_idx(110, 300001, 5000)), ("src", data(F32, (300001,), 111))], "scatter_direct"),
    ("scatter_slice_lds=131072,scatter_slice_bins=32768", lambda: C.scatter_gather(300001, 1 << 18, F32),
     lambda: [("idx", scatter_idx(112, 300001, 1 << 18)), ("src", data(F32, (300001,), 113))], "gather_unpartition"),
    ("scatter_slice_wgs=64", lambda: C.scatter_gather(300001, 70000, F32),
     lambda: [("idx", scatter_idx(114, 300001, 70000)), ("src", data(F32, (300001,), 115))], "scatter_accumulate"),
    ("scatter_stage_p=8", lambda: C.scatter_gather(300001, 1 << 18, F32),
     lambda: [("idx", scatter_idx(116, 300001, 1 << 18)), ("src", data(F32, (300001,), 117))], "scatter_coarse"),
    ("scatter_tile=4096", lambda: C.scatter_gather(300001, 70000, F32),
     lambda: [("idx", scatter_idx(118, 300001, 70000)), ("src", data(F32, (300001,), 119))], "scatter_partition"),
    # split-k taken at a shorter k, and refused
    ("mm_splitk_min_k=1024", lambda: C.matmul(3, F64, k=2048, m=3),
     lambda: [("a", data(F64, (3, 2048), 120)), ("b", data(F64, (2048, 3), 121))], "matmul_splitk"),
    ("mm_splitk_outputs=0", lambda: C.matmul(3, F64, k=65536, m=3),
     lambda: [("a", data(F64, (3, 65536), 122)), ("b", data(F64, (65536, 3), 123))], "matmul_tiled"),
    # a one-kernel program replayed from a recorded HIP graph
    ("graphs=1,graph_min_kernels=1", lambda: P.chain(5000).graph(), lambda: P.chain(5000).inputs(), "map"),
    # the lowering's own rewrites turned off, each on a graph that takes it
    ("same_fold=0", lambda: _pair_graph(), lambda: [("x", data(F32, (2048, 300), 124))], "reduce_rowseq"),
    ("fuse_reduce_expr=0", lambda: _expr_sum_graph(True), lambda: _expr_sum_inputs(125), "reduce_split"),
    ("skip_unread_stores=0", lambda: _expr_sum_graph(False), lambda: _expr_sum_inputs(126), "map"),
    ("scatter_inline=0", lambda: _affine_read_graph(), lambda: _affine_read_inputs(127), "scatter_affine"),
    ("map_unroll_gx=0", lambda: _exp_gather_graph(), lambda: _exp_gather_inputs(128), "map"),
]


def _pair_graph():
    x, z = D.param("x", F32, (2048, 300)), D.const(F32, 0.0)
    return Graph.create("pair", [("s", D.scan_rows(D.add, z, x)), ("r", D.reduce_rows(D.add, z, x))])


def _expr_sum_graph(out):
    n = 300001
    x, y, z = (D.param(c, F32, (n,)) for c in "xyz")
    a = D.map2(lambda u, v: D.add(D.mul(u, D.const(F32, 2.0)), v), x, y)
    e = D.map2(D.mul, a, z) if out else D.map2(D.add, D.map2(D.mul, a, z), a)
    return Graph.create("esum", ([("a", a)] if out else []) + [("s", D.reduce(D.max, D.const(F32, -1e30), e))])


def _expr_sum_inputs(seed):
    return [(c, data(F32, (300001,), seed + k)) for k, c in enumerate("xyz")]


def _affine_read_graph():
    n = 100003
    idx = D.map(lambda p: D.add(D.mul(p, D.const(I32, 64)), D.const(I32, 63)), D.iota((n,)))
    h = D.scatter_add(idx, D.param("src", F32, (n,)), (64 * n,))
    return Graph.create("aread", [("o", D.map2(D.mul, h, D.param("y", F32, (64 * n,))))])


def _affine_read_inputs(seed):
    return [("src", data(F32, (100003,), seed)), ("y", data(F32, (64 * 100003,), seed + 1))]


def _exp_gather_graph():
    n = 300001
    x, y, gi = D.param("x", F32, (n,)), D.param("y", F32, (n,)), D.param("gi", I32, (n,))
    return Graph.create("eg", [("o", D.map2(lambda u, v: D.mul(D.exp(u), v), x, D.gather(gi, y)))])


def _exp_gather_inputs(seed):
    n = 300001
    return [("x", data(F32, (n,), seed)), ("y", data(F32, (n,), seed + 1)),
            ("gi", np.random.default_rng(seed).integers(0, n, size=n).astype(np.int32))]


@pytest.mark.parametrize("knob,graph,inputs,tpl", KNOB_CASES, ids=[c[0] for c in KNOB_CASES])
def test_tuning_knobs_keep_results(device, monkeypatch, knob, graph, inputs, tpl):
    """A CCHIP_TUNE setting changes launch shapes or tiling, never what is
    computed: every non-default path against the oracle."""
    monkeypatch.setenv("CCHIP_TUNE", knob)
    check(graph(), inputs(), [tpl])
