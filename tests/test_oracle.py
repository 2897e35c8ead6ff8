"""Pins the CPU oracle (oracle/interp.c) before anything is judged by it.

Every expected value here comes from the reference's own tests (file:line
cited on each case), from a published known-answer vector, or from an
independent computation (numpy's IEEE float32 arithmetic, math.erf, a
brute-force search) chosen so that a plausible mistake in the restatement
fails: a rounded F32 constant, a fused multiply-add, a non-sequential fold,
a NaN-dropping min, a saturating cast. None of them is produced by the code
under test. No GPU needed."""

import math

import numpy as np
import pytest

import oracle
from cudacaml_amd import dsl as D
from cudacaml_amd import rng
from cudacaml_amd.examples import configs as C
from cudacaml_amd.examples import programs as P
from cudacaml_amd.ir import F32, F64, I32, I64, Graph

run = oracle.run


def vec(n):
    return (n,)


def f32(l):
    return np.array(l, dtype=np.float32)


def f64(l):
    return np.array(l, dtype=np.float64)


def i32(l):
    return np.array(l, dtype=np.int32)


def i64(l):
    return np.array(l, dtype=np.int64)


def out(o, name):
    return dict(o)[name]


def one(name, t):
    return Graph.create("g", [(name, t)])


# ---------------------------------------------------------------------------
# test/unit/test_interp.ml:28-120 (hand-computed values)
# ---------------------------------------------------------------------------


def test_interp_map():
    x = D.param("x", F32, vec(3))
    g = one("r", D.map(lambda e: D.mul(e, e), x))
    assert out(run(g, [("x", f32([1, 2, 3]))]), "r").tolist() == [1, 4, 9]


def test_interp_map2_fused_chain():
    x, y = D.param("x", F32, vec(3)), D.param("y", F32, vec(3))
    r = D.map2(D.add, D.map(lambda e: D.mul(D.const(F32, 2.0), e), x), y)
    o = run(one("r", r), [("x", f32([1, 2, 3])), ("y", f32([10, 20, 30]))])
    assert out(o, "r").tolist() == [12, 24, 36]


def test_interp_iota_cast_and_index():
    assert out(run(one("r", D.map(lambda i: D.cast(F32, i), D.iota(vec(4)))), []), "r").tolist() == [0, 1, 2, 3]
    x = D.param("x", F32, vec(3))
    g = one("r", D.map(lambda e: D.add(e, D.cast(F32, D.index())), x))
    assert out(run(g, [("x", f32([10, 10, 10]))]), "r").tolist() == [10, 11, 12]


def test_interp_reduce_fold_from_init_max_empty():
    x = D.param("x", F32, vec(4))
    assert out(run(one("s", D.reduce(D.add, D.const(F32, 100.0), x)), [("x", f32([1, 2, 3, 4]))]), "s") == 110
    x = D.param("x", F32, vec(3))
    assert out(run(one("m", D.reduce(D.max, D.const(F32, -1e30), x)), [("x", f32([-3, 7, 2]))]), "m") == 7
    x = D.param("x", F32, vec(0))
    assert out(run(one("s", D.reduce(D.add, D.const(F32, 5.0), x)), [("x", f32([]))]), "s") == 5


def test_interp_scan_gather_reshape_select():
    x = D.param("x", F32, vec(4))
    assert out(run(one("p", D.scan(D.add, D.const(F32, 0.0), x)), [("x", f32([1, 2, 3, 4]))]), "p").tolist() == [1, 3, 6, 10]
    x, i = D.param("x", F32, vec(3)), D.param("i", I32, vec(4))
    o = run(one("r", D.gather(i, x)), [("x", f32([10, 20, 30])), ("i", i32([2, 0, 2, 1]))])
    assert out(o, "r").tolist() == [30, 10, 30, 20]
    x = D.param("x", F32, (2, 2))
    r = out(run(one("r", D.reshape(vec(4), x)), [("x", f32([[1, 2], [3, 4]]))]), "r")
    assert r.tolist() == [1, 2, 3, 4] and r.shape == (4,)
    x = D.param("x", F32, vec(4))
    z = D.const(F32, 0.0)
    g = one("r", D.map(lambda e: D.select(D.lt(e, z), z, e), x))
    assert out(run(g, [("x", f32([-1, 2, -3, 4]))]), "r").tolist() == [0, 2, 0, 4]


def test_interp_gather_out_of_bounds_raises():
    x, i = D.param("x", F32, vec(3)), D.param("i", I32, vec(1))
    with pytest.raises(oracle.OracleError, match="gather index out of bounds"):
        run(one("r", D.gather(i, x)), [("x", f32([1, 2, 3])), ("i", i32([3]))])


def test_interp_i32_division_truncates():
    x = D.param("x", I32, vec(2))
    g = one("r", D.map(lambda e: D.div(e, D.const(I32, 2)), x))
    assert out(run(g, [("x", i32([-7, 7]))]), "r").tolist() == [-3, 3]


def test_interp_f32_rounding():
    x = D.param("x", F32, vec(1))
    g = one("r", D.map(lambda e: D.add(e, D.const(F32, 0.2)), x))
    v = float(out(run(g, [("x", f32([0.1]))]), "r")[0])
    assert abs(v - 0.300000011920929) <= 1e-9


def test_interp_shared_intermediate_and_output_order():
    x = D.param("x", F32, vec(2))
    s = D.map(lambda e: D.mul(e, e), x)
    g = Graph.create("g", [("a", D.map(D.neg, s)), ("c", D.reduce(D.add, D.const(F32, 0.0), s))])
    o = run(g, [("x", f32([3, 4]))])
    assert [n for n, _ in o] == ["a", "c"]
    assert out(o, "a").tolist() == [-9, -16] and out(o, "c") == 25


@pytest.mark.parametrize("inputs", [[], [("x", f32([1.0]))], [("x", i32([1]))]],
                         ids=["missing", "wrong-shape", "wrong-dtype"])
def test_interp_bad_inputs_raise(inputs):
    x = D.param("x", F32, vec(2) if inputs and inputs[0][1].dtype == np.float32 else vec(1))
    with pytest.raises(oracle.OracleError):
        run(one("r", D.map(D.neg, x)), inputs)


def test_every_example_runs():
    for e in P.all_examples():
        run(e.graph(), e.inputs())


# ---------------------------------------------------------------------------
# test/unit/test_rng.ml:71-129 (Random123 known-answer vectors, statistics)
# ---------------------------------------------------------------------------

KATS = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,expect", KATS, ids=["zero", "ones", "pi"])
def test_philox_kat_through_graph(ctr, key, expect):
    k = lambda v: D.const(I32, v)  # noqa: E731
    x = D.param("x", I32, vec(1))
    outs = []
    for w in range(4):
        outs.append(("w%d" % w, D.map(lambda _, w=w: rng.round10(tuple(k(c) for c in ctr), (k(key[0]), k(key[1])))[w], x)))
    o = run(Graph.create("kat", outs), [("x", i32([0]))])
    got = tuple(int(v[0]) & 0xFFFFFFFF for _, v in o)
    assert got == expect


@pytest.mark.parametrize("ctr,key,expect", KATS, ids=["zero", "ones", "pi"])
def test_philox_kat_host_generators(ctr, key, expect):
    assert tuple(oracle.philox4x32_10(ctr, key)) == expect
    if ctr[1:] == (0, 0, 0) and key[1] == 0:
        assert int(C.philox_w0(key[0], 1, start=ctr[0])[0]) == expect[0]


def u32_list(key, n):
    g = one("r", rng.u32(D.scalar("seed", I32), vec(n)))
    return out(run(g, [("seed", np.array(key, dtype=np.int32))]), "r")


def test_u32_element0_and_reproducible():
    l = u32_list(0, 4)
    assert int(l[0]) & 0xFFFFFFFF == 0x6627E8D5 and len(set(l.tolist())) == 4
    a, b, c = u32_list(42, 1024), u32_list(42, 1024), u32_list(43, 1024)
    assert (a == b).all() and int((a != c).sum()) >= 922


def test_u32_matches_host_generator():
    n = 4096
    np.testing.assert_array_equal(u32_list(9, n).view(np.uint32), C.philox_w0(9, n))


def test_uniform_f64_statistics():
    n = 65536
    u = out(run(one("r", rng.uniform(F64, D.scalar("seed", I32), vec(n))), [("seed", np.array(1, np.int32))]), "r")
    assert ((u > 0) & (u < 1)).all()
    assert abs(u.mean() - 0.5) <= 0.01 and abs(u.var() - 1 / 12) <= 0.005
    counts = np.bincount((u * 16).astype(int), minlength=16)
    e = n / 16
    assert ((counts - e) ** 2 / e).sum() < 45.0


def test_normal_statistics():
    n = 65536
    z = out(run(one("r", rng.normal(F64, D.scalar("seed", I32), vec(n))), [("seed", np.array(2, np.int32))]), "r")
    assert np.isfinite(z).all() and abs(z.mean()) <= 0.02 and abs(z.var() - 1) <= 0.05
    assert abs((np.abs(z) > 1.96).mean() - 0.05) <= 0.006
    z32 = out(run(one("r", rng.normal(F32, D.scalar("seed", I32), vec(n))), [("seed", np.array(3, np.int32))]), "r")
    assert np.isfinite(z32).all() and abs(z32.mean()) <= 0.02


def test_counter_is_flat_index():
    k = lambda: D.scalar("seed", I32)  # noqa: E731
    a = out(run(one("r", rng.u32(k(), (4, 8))), [("seed", np.array(9, np.int32))]), "r")
    b = out(run(one("r", rng.u32(k(), vec(32))), [("seed", np.array(9, np.int32))]), "r")
    np.testing.assert_array_equal(a.reshape(-1), b)


# ---------------------------------------------------------------------------
# test/unit/test_expr_ops.ml:49-119
# ---------------------------------------------------------------------------


def binop32(f, xs, ys):
    x, y = D.param("x", I32, vec(len(xs))), D.param("y", I32, vec(len(ys)))
    return out(run(one("r", D.map2(f, x, y)), [("x", i32(xs)), ("y", i32(ys))]), "r").tolist()


def binop64(f, xs, ys):
    x, y = D.param("x", I64, vec(len(xs))), D.param("y", I64, vec(len(ys)))
    return out(run(one("r", D.map2(f, x, y)), [("x", i64(xs)), ("y", i64(ys))]), "r").tolist()


def h(v):
    return v - (1 << 32) if v >= (1 << 31) else v


def test_i32_bit_ops():
    a, b = [0x0F0F0F0F], [0x00FF00FF]
    assert binop32(D.bit_xor, a, b) == [0x0FF00FF0]
    assert binop32(D.bit_and, a, b) == [0x000F000F]
    assert binop32(D.bit_or, a, b) == [0x0FFF0FFF]
    assert binop32(D.bit_xor, [-1], [5]) == [-6]
    assert binop32(D.bit_and, [-8], [255]) == [248]
    assert binop32(D.bit_or, [-8], [3]) == [-5]


def test_shifts_logical_masked():
    assert binop32(D.shl, [1], [31]) == [-(1 << 31)]
    assert binop32(D.shr, [-1], [28]) == [15]
    assert binop32(D.shr, [12345], [32]) == [12345]
    assert binop32(D.shl, [3], [33]) == [6]
    assert binop32(D.shr, [-(1 << 31)], [31]) == [1]
    assert binop64(D.shr, [-1], [60]) == [15]
    assert binop64(D.shl, [1], [63]) == [-(1 << 63)]


def test_bit_ops_on_floats_rejected():
    x = D.param("x", F32, vec(1))
    with pytest.raises(oracle.OracleError):
        run(one("r", D.map2(D.bit_and, x, x)), [("x", f32([1.0]))])


def unop_f64(f, xs):
    x = D.param("x", F64, vec(len(xs)))
    return out(run(one("r", D.map(f, x)), [("x", f64(xs))]), "r")


def test_sin_cos_erf_f64():
    pi2 = math.pi / 2
    np.testing.assert_allclose(unop_f64(D.sin, [0.0, pi2]), [0, 1], atol=1e-12)
    np.testing.assert_allclose(unop_f64(D.cos, [0.0, pi2]), [1, 0], atol=1e-12)
    np.testing.assert_allclose(unop_f64(D.erf, [0.0, 1.0]), [0, 0.8427007929497149], atol=1e-15)


def test_erfinv_inverts_erf_and_edges():
    xs = [-2.0, -0.5, 0.0, 0.3, 1.5, 2.5]
    np.testing.assert_allclose(unop_f64(lambda e: D.erfinv(D.erf(e)), xs), xs, atol=1e-12 * 3.5)
    p, z, m = unop_f64(D.erfinv, [1.0, 0.0, -1.0])
    assert p == math.inf and z == 0.0 and m == -math.inf
    # erfinv(0.5) from tables; and erf of the oracle's answer returns the input.
    assert abs(oracle.erfinv(0.5) - 0.4769362762044699) < 1e-15
    for y in np.linspace(-0.999, 0.999, 41):
        assert abs(math.erf(oracle.erfinv(float(y))) - y) < 2e-16 * 8


def test_erfinv_f32():
    x = D.param("x", F32, vec(1))
    v = float(out(run(one("r", D.map(D.erfinv, x)), [("x", f32([0.5]))]), "r")[0])
    assert abs(v - 0.4769362762) <= 1e-6


def test_comparisons_and_logic_through_select():
    x, y = D.param("x", F32, vec(3)), D.param("y", F32, vec(3))
    b = lambda c: D.select(c, D.const(F32, 1.0), D.const(F32, 0.0))  # noqa: E731
    k = lambda v: D.const(F32, v)  # noqa: E731
    g = Graph.create("g", [
        ("ne", D.map2(lambda a, c: b(D.ne(a, c)), x, y)),
        ("gt", D.map2(lambda a, c: b(D.gt(a, c)), x, y)),
        ("ge", D.map2(lambda a, c: b(D.ge(a, c)), x, y)),
        ("and", D.map(lambda a: b(D.and_(D.gt(a, k(1.0)), D.lt(a, k(3.0)))), x)),
        ("or", D.map(lambda a: b(D.or_(D.lt(a, k(2.0)), D.gt(a, k(2.0)))), x)),
        ("not", D.map2(lambda a, c: b(D.not_(D.eq(a, c))), x, y)),
    ])
    o = dict(run(g, [("x", f32([1, 2, 3])), ("y", f32([2, 2, 2]))]))
    assert o["ne"].tolist() == [1, 0, 1] and o["gt"].tolist() == [0, 0, 1] and o["ge"].tolist() == [0, 1, 1]
    assert o["and"].tolist() == [0, 1, 0] and o["or"].tolist() == [1, 0, 1] and o["not"].tolist() == [1, 0, 1]


# ---------------------------------------------------------------------------
# Rules the reference tests leave open, pinned independently
# ---------------------------------------------------------------------------


def test_r1_f32_ops_match_ieee_single():
    """R1: every F32 op rounds once; numpy float32 arithmetic is IEEE single."""
    rs = np.random.default_rng(0)
    a = (rs.standard_normal(4096) * 10 ** rs.uniform(-3, 3, 4096)).astype(np.float32)
    b = (rs.standard_normal(4096) * 10 ** rs.uniform(-3, 3, 4096)).astype(np.float32)
    x, y = D.param("x", F32, vec(4096)), D.param("y", F32, vec(4096))
    for f, ref in [(D.add, a + b), (D.sub, a - b), (D.mul, a * b), (D.div, a / b)]:
        got = out(run(one("r", D.map2(f, x, y)), [("x", a), ("y", b)]), "r")
        np.testing.assert_array_equal(got, ref)
    got = out(run(one("r", D.map(D.sqrt, x)), [("x", np.abs(a))]), "r")
    np.testing.assert_array_equal(got, np.sqrt(np.abs(a)))


def test_r1_no_fused_multiply_add():
    """a*b + c rounds the product first: a case where fma differs."""
    a = np.float32(1.0 + 2.0 ** -12)
    c = np.float32(-(1.0 + 2.0 ** -11))
    x, y = D.param("x", F32, vec(1)), D.param("y", F32, vec(1))
    got = out(run(one("r", D.map2(lambda u, v: D.add(D.mul(u, u), v), x, y)), [("x", f32([a])), ("y", f32([c]))]), "r")
    rounded = np.float32(np.float32(a * a) + c)
    fused = np.float32(float(a) * float(a) + float(c))
    assert rounded != fused and got[0] == rounded


def test_r3_f32_constant_is_the_unrounded_double():
    """An F32 Const is the OCaml double (interp.ml:246): x * c rounds
    x*c_double once. Find inputs where rounding c first would differ."""
    c = 0.1
    xs = np.arange(1, 200000, dtype=np.float32) * np.float32(1.0009765625)
    exact = (xs.astype(np.float64) * c).astype(np.float32)
    pre = xs * np.float32(c)
    diff = np.nonzero(exact != pre)[0][:64]
    assert len(diff) > 0
    x = D.param("x", F32, vec(len(diff)))
    got = out(run(one("r", D.map(lambda e: D.mul(e, D.const(F32, c)), x)), [("x", xs[diff])]), "r")
    np.testing.assert_array_equal(got, exact[diff])


def test_r5_min_max_nan_and_signed_zero():
    """OCaml Float.min/max: NaN if either is NaN, min(-0,+0) = -0."""
    x, y = D.param("x", F64, vec(4)), D.param("y", F64, vec(4))
    xs, ys = f64([math.nan, 1.0, -0.0, 0.0]), f64([1.0, math.nan, 0.0, -0.0])
    o = dict(run(Graph.create("g", [("mn", D.map2(D.min, x, y)), ("mx", D.map2(D.max, x, y))]), [("x", xs), ("y", ys)]))
    assert np.isnan(o["mn"][:2]).all() and np.isnan(o["mx"][:2]).all()
    assert math.copysign(1, o["mn"][2]) == -1 and math.copysign(1, o["mn"][3]) == -1
    assert math.copysign(1, o["mx"][2]) == 1 and math.copysign(1, o["mx"][3]) == 1


def test_r6_float_to_int_casts_wrap():
    x = D.param("x", F64, vec(5))
    o = out(run(one("r", D.map(lambda e: D.cast(I32, e), x)), [("x", f64([3e9, -2.7, 2.7, -3e9, 2 ** 31]))]), "r")
    assert o.tolist() == [3000000000 - (1 << 32), -2, 2, -3000000000 + (1 << 32), -(1 << 31)]
    y = D.param("y", I64, vec(1))
    o = out(run(one("r", D.map(lambda e: D.cast(F32, e), y)), [("y", i64([(1 << 53) + 1]))]), "r")
    assert o[0] == np.float32(float((1 << 53) + 1))


def test_r2_reduce_and_scan_are_sequential_folds():
    vals = f32([1e8, 1.0, 1.0, 1.0, 1.0, -1e8, 1.0])
    x = D.param("x", F32, vec(7))
    seq = np.float32(0)
    pref = []
    for v in vals:
        seq = np.float32(seq + v)
        pref.append(seq)
    o = dict(run(Graph.create("g", [("s", D.reduce(D.add, D.const(F32, 0.0), x)),
                                    ("p", D.scan(D.add, D.const(F32, 0.0), x))]), [("x", vals)]))
    assert o["s"] == seq == np.float32(1.0)
    np.testing.assert_array_equal(o["p"], f32(pref))


def test_r8_scatter_is_sequential_in_source_order():
    idx = D.param("idx", I32, vec(4))
    src = D.param("src", F32, vec(4))
    o = run(one("h", D.scatter_add(idx, src, vec(1))), [("idx", i32([0, 0, 0, 0])), ("src", f32([1e8, 1, -1e8, 1]))])
    assert out(o, "h").tolist() == [1.0]


def test_r9_matmul_rounds_product_then_sum():
    a = f32([[1.0 + 2.0 ** -12, 1.0]])
    b = f32([[1.0 + 2.0 ** -12], [-(1.0 + 2.0 ** -11)]])
    A, B = D.param("a", F32, (1, 2)), D.param("b", F32, (2, 1))
    got = out(run(one("c", D.matmul(A, B)), [("a", a), ("b", b)]), "c")
    acc = np.float32(0)
    for p in range(2):
        acc = np.float32(acc + np.float32(a[0, p] * b[p, 0]))
    assert got[0, 0] == acc


# ---------------------------------------------------------------------------
# test/unit/test_rows.ml:45-80, test_scatter.ml:34-46, test_matmul.ml:91-103
# ---------------------------------------------------------------------------

IN23 = f32([[1, 2, 3], [4, 5, 6]])


def test_rows_reduce_scan_transpose():
    x = D.param("x", F32, (2, 3))
    z = D.const(F32, 0.0)
    r = out(run(one("r", D.reduce_rows(D.add, z, x)), [("x", IN23)]), "r")
    assert r.tolist() == [6, 15] and r.shape == (2,)
    s = out(run(one("s", D.reduce(D.add, z, x)), [("x", IN23)]), "s")
    assert s == 21 and s.shape == ()
    x = D.param("x", F32, (2, 3))
    o = dict(run(Graph.create("g", [("rows", D.scan_rows(D.add, z, x)), ("flat", D.scan(D.add, z, x))]), [("x", IN23)]))
    assert o["rows"].reshape(-1).tolist() == [1, 3, 6, 4, 9, 15] and o["rows"].shape == (2, 3)
    assert o["flat"].reshape(-1).tolist() == [1, 3, 6, 10, 15, 21] and o["flat"].shape == (2, 3)
    x = D.param("x", F32, (2, 3))
    assert out(run(one("m", D.reduce_rows(D.max, D.const(F32, -1e30), x)), [("x", IN23)]), "m").tolist() == [3, 6]
    x = D.param("x", F32, (2, 3))
    o = dict(run(Graph.create("g", [("t", D.transpose(x)), ("cols", D.reduce_rows(D.add, z, D.transpose(x)))]),
                 [("x", IN23)]))
    assert o["t"].reshape(-1).tolist() == [1, 4, 2, 5, 3, 6] and o["t"].shape == (3, 2)
    assert o["cols"].tolist() == [5, 7, 9]


def test_scatter_histograms_and_errors():
    idx6 = i32([0, 1, 1, 3, 3, 3])
    idx, src = D.param("idx", I32, vec(6)), D.param("src", F32, vec(6))
    o = run(one("h", D.scatter_add(idx, src, vec(4))), [("idx", idx6), ("src", np.ones(6, np.float32))])
    assert out(o, "h").tolist() == [1, 2, 0, 3]
    idx, src = D.param("idx", I32, vec(6)), D.param("src", I32, vec(6))
    o = run(one("h", D.scatter_add(idx, src, vec(4))), [("idx", idx6), ("src", i32([1, 2, 3, 4, 5, 6]))])
    assert out(o, "h").tolist() == [1, 5, 0, 15]
    idx, src = D.param("idx", I32, vec(1)), D.param("src", F32, vec(1))
    with pytest.raises(oracle.OracleError, match="scatter_add index out of bounds"):
        run(one("h", D.scatter_add(idx, src, vec(4))), [("idx", i32([4])), ("src", f32([1.0]))])


def mm(m, k, n, a, b):
    A, B = D.param("a", F64, (m, k)), D.param("b", F64, (k, n))
    o = run(one("c", D.matmul(A, B)), [("a", f64(a).reshape(m, k)), ("b", f64(b).reshape(k, n))])
    return out(o, "c")


def test_matmul_values():
    c = mm(2, 3, 2, [1, 2, 3, 4, 5, 6], [7, 8, 9, 10, 11, 12])
    assert c.reshape(-1).tolist() == [58, 64, 139, 154] and c.shape == (2, 2)
    a = list(range(1, 10))
    assert mm(3, 3, 3, a, [1, 0, 0, 0, 1, 0, 0, 0, 1]).reshape(-1).tolist() == a
    av = [((i * 7) % 11) - 5.0 for i in range(35)]
    bv = [((i * 5) % 13) / 4.0 for i in range(21)]
    ref = np.array(av).reshape(5, 7) @ np.array(bv).reshape(7, 3)
    np.testing.assert_allclose(mm(5, 7, 3, av, bv), ref, rtol=0, atol=1e-12)


# ---------------------------------------------------------------------------
# test/unit/test_grad.ml and test_matmul.ml:64-88: gradients against central
# differences of the ORIGINAL graph, both run on the oracle.
# ---------------------------------------------------------------------------

from cudacaml_amd import grad as G  # noqa: E402


def fd(g, output, wrt, inputs, hstep=1e-6):
    base = dict(inputs)[wrt]
    res = np.zeros(base.size)
    for i in range(base.size):
        vals = []
        for d in (hstep, -hstep):
            v = base.copy().reshape(-1)
            v[i] += d
            ins = [(n, v.reshape(base.shape) if n == wrt else x) for n, x in inputs]
            vals.append(float(np.sum(out(run(g, ins), output))))
        res[i] = (vals[0] - vals[1]) / (2 * hstep)
    return res


def grad_vs_fd(g, output, wrt, inputs, tol=1e-5):
    gg = G.grad(g, output, wrt)
    o = dict(run(gg, inputs))
    for w in wrt:
        e = fd(g, output, w, inputs)
        got = o[G.grad_name(output, w)].reshape(-1)
        assert np.all(np.abs(e - got) <= tol * (1 + np.abs(e))), (w, e, got)
    return o


XS4 = f64([1.0, -2.0, 0.5, 3.0])
YS4 = f64([0.3, 1.5, -1.0, 2.0])


def p64(name, dims):
    return D.param(name, F64, dims)


def test_grad_basic_rules():
    x = p64("x", vec(4))
    g = one("s", D.reduce(D.add, D.const(F64, 0.0), D.map(lambda e: D.mul(e, e), x)))
    o = grad_vs_fd(g, "s", ["x"], [("x", XS4)])
    np.testing.assert_allclose(o["ds/dx"], 2 * XS4, atol=1e-9)
    x, y = p64("x", vec(4)), p64("y", vec(4))
    g = one("s", D.reduce(D.add, D.const(F64, 0.0), D.map2(D.mul, x, y)))
    o = grad_vs_fd(g, "s", ["x", "y"], [("x", XS4), ("y", YS4)])
    np.testing.assert_allclose(o["ds/dx"], YS4, atol=1e-9)
    np.testing.assert_allclose(o["ds/dy"], XS4, atol=1e-9)
    x, y = p64("x", vec(4)), p64("y", vec(4))
    r = D.map2(lambda a, b: D.add(D.mul(D.exp(a), b), D.sin(D.mul(a, b))), x, y)
    grad_vs_fd(one("s", D.reduce(D.add, D.const(F64, 0.0), r)), "s", ["x", "y"], [("x", XS4), ("y", YS4)])


def test_grad_reductions_and_scans():
    x = p64("x", vec(4))
    o = grad_vs_fd(one("m", D.reduce(D.max, D.const(F64, -1e300), x)), "m", ["x"], [("x", f64([1, 5, 3, 2]))])
    assert o["dm/dx"].tolist() == [0, 1, 0, 0]
    x, w = p64("x", (2, 3)), p64("w", vec(2))
    z = D.const(F64, 0.0)
    g = one("s", D.reduce(D.add, z, D.map2(D.mul, w, D.reduce_rows(D.add, z, x))))
    o = grad_vs_fd(g, "s", ["x", "w"], [("x", f64([[1, 2, 3], [4, 5, 6]])), ("w", f64([10, 20]))])
    assert o["ds/dx"].reshape(-1).tolist() == [10, 10, 10, 20, 20, 20] and o["ds/dx"].shape == (2, 3)
    x, w = p64("x", vec(4)), p64("w", vec(4))
    g = one("s", D.reduce(D.add, z, D.map2(D.mul, w, D.scan(D.add, z, x))))
    o = grad_vs_fd(g, "s", ["x"], [("x", XS4), ("w", YS4)])
    np.testing.assert_allclose(o["ds/dx"], [2.8, 2.5, 1.0, 2.0], atol=1e-9)
    x, w = p64("x", (2, 3)), p64("w", (2, 3))
    g = one("s", D.reduce(D.add, z, D.map2(D.mul, w, D.scan_rows(D.add, z, x))))
    v = f64([[1, 2, 3], [4, 5, 6]])
    o = grad_vs_fd(g, "s", ["x"], [("x", v), ("w", v)])
    np.testing.assert_allclose(o["ds/dx"].reshape(-1), [6, 5, 3, 15, 11, 6], atol=1e-9)


def test_grad_broadcast_reshape_gather_unused():
    z = D.const(F64, 0.0)
    x, s = p64("x", vec(4)), D.scalar("s", F64)
    g = one("t", D.reduce(D.add, z, D.map2(D.mul, x, D.broadcast(vec(4), s))))
    o = grad_vs_fd(g, "t", ["s", "x"], [("x", XS4), ("s", np.array(1.7))])
    assert abs(float(o["dt/ds"]) - XS4.sum()) < 1e-9 and o["dt/ds"].shape == ()
    x = p64("x", (2, 3))
    g = one("s", D.reduce(D.add, z, D.map(lambda e: D.mul(e, e), D.reshape(vec(6), x))))
    o = grad_vs_fd(g, "s", ["x"], [("x", f64([[1, 2, 3], [4, 5, 6]]))])
    assert o["ds/dx"].shape == (2, 3)
    x, idx = p64("x", vec(3)), D.param("idx", I32, vec(3))
    g = one("s", D.reduce(D.add, z, D.gather(idx, x)))
    o = grad_vs_fd(g, "s", ["x"], [("x", f64([1, 2, 3])), ("idx", i32([0, 0, 1]))])
    assert o["ds/dx"].tolist() == [2, 1, 0]
    x, y = p64("x", vec(4)), p64("y", (2, 2))
    g = Graph.create("g", [("s", D.reduce(D.add, z, x)), ("y", y)])
    o = dict(run(G.grad(g, "s", ["y"]), [("x", XS4), ("y", YS4.reshape(2, 2))]))
    assert o["ds/dy"].tolist() == [[0, 0], [0, 0]]
    x = p64("x", vec(4))
    with pytest.raises(G.NotDifferentiable, match="Reduce"):
        G.grad(one("s", D.reduce(lambda a, b: D.add(D.mul(a, b), a), z, x)), "s", ["x"])


def test_grad_matmul_closed_form_and_fd():
    """d sum(AB)/dA[i,p] = sum_j B[p,j]; d/dB[p,j] = sum_i A[i,p]."""
    a, b = p64("a", (2, 3)), p64("b", (3, 2))
    av = f64([[1, -2, 0.5], [3, 1.5, -1]])
    bv = f64([[0.3, 1.5], [-1, 2], [0.7, -0.2]])
    g = one("s", D.reduce(D.add, D.const(F64, 0.0), D.matmul(a, b)))
    o = grad_vs_fd(g, "s", ["a", "b"], [("a", av), ("b", bv)])
    np.testing.assert_allclose(o["ds/da"], np.tile(bv.sum(axis=1), (2, 1)), atol=1e-12)
    np.testing.assert_allclose(o["ds/db"], np.tile(av.sum(axis=0)[:, None], (1, 2)), atol=1e-12)
    a, b = p64("a", (2, 3)), p64("b", (3, 2))
    g = one("s", D.reduce(D.add, D.const(F64, 0.0), D.matmul(D.map(D.exp, a), b)))
    grad_vs_fd(g, "s", ["a", "b"], [("a", av), ("b", bv)])


# ---------------------------------------------------------------------------
# test/unit/test_black_scholes.ml:13-41
# ---------------------------------------------------------------------------

from cudacaml_amd.examples import black_scholes as bs  # noqa: E402


def test_black_scholes_closed_form_and_mc():
    cf = bs.analytic()
    assert abs(cf["price"] - 10.4506) <= 2e-3 and abs(cf["delta"] - 0.6368) <= 2e-3
    assert abs(cf["vega"] - 37.524) <= 2e-3 and abs(cf["rho"] - 53.232) <= 2e-3
    ins = bs.inputs(F64, seed=7)
    price = bs.scalar_out(run(bs.call_mc(65536, F64), ins), "price")
    assert abs(price - cf["price"]) <= 0.25
    assert abs(bs.scalar_out(run(bs.call_mc_paths(16384, 8, F64), ins), "price") - cf["price"]) <= 0.5
    o = run(bs.call_greeks(65536, F64), ins)
    assert bs.scalar_out(o, "price") == price
    assert abs(bs.scalar_out(o, "dprice/ds0") - cf["delta"]) <= 0.02
    assert abs(bs.scalar_out(o, "dprice/dvol") - cf["vega"]) <= 1.5
    assert abs(bs.scalar_out(o, "dprice/drate") - cf["rho"]) <= 1.5


def test_paths_greeks_pathwise_estimator():
    """delta and vega of the multi-step pricer against the hand-derived
    pathwise estimator on the same Philox draws (exact GBM):
    delta = e^-rT mean(1{S_T>K} S_T/S0), vega = e^-rT mean(1{S_T>K} S_T (sqrt(dt) sum Z - vol T))."""
    n, steps = 4096, 8
    m = bs.market
    ins = bs.inputs(F64, seed=7)
    o = dict(run(bs.call_paths_greeks(n, steps, F64), ins))
    zg = one("z", rng.normal(F64, D.scalar("seed", I32), (n, steps)))
    z = out(run(zg, [("seed", np.array(7, np.int32))]), "z")
    dt = m.maturity / steps
    logs = np.log(m.s0) + np.cumsum((m.rate - 0.5 * m.vol ** 2) * dt + m.vol * math.sqrt(dt) * z, axis=1)
    st = np.exp(logs[:, -1])
    itm = st > m.strike
    disc = math.exp(-m.rate * m.maturity)
    delta = disc * np.mean(itm * st / m.s0)
    vega = disc * np.mean(itm * st * (math.sqrt(dt) * z.sum(axis=1) - m.vol * m.maturity))
    assert abs(float(o["dprice/ds0"]) - delta) <= 1e-9 * (1 + abs(delta))
    assert abs(float(o["dprice/dvol"]) - vega) <= 1e-9 * (1 + abs(vega))


def test_greeks_graph_shape():
    g = bs.call_greeks(4096, F64)
    assert sorted(n for n, _ in g.params) == ["rate", "s0", "seed", "vol"]
    assert len(g.outputs) == 4


# ---------------------------------------------------------------------------
# bench/bench.ml:70-126 (the reference benchmark's graphs): the degree-64
# Horner chain against an independent numpy restatement of R1/R3 (each
# product rounded to single, each f32 constant added as the unrounded
# double, then rounded), and the f64 chain against plain float64 Horner.
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", [F32, F64], ids=["f32", "f64"])
def test_refbench_poly_horner(dtype):
    from cudacaml_amd.examples import refbench as RB

    n = 4096
    x = RB.x_input(n, dtype)
    o = dict(run(RB.poly_graph(n, dtype), [("x", x)]))
    c = RB.coefficients()
    assert len(c) == 64 and c[2] == 1.0 / 3.0
    with np.errstate(over="ignore", invalid="ignore"):
        if dtype is F32:
            acc = np.full(n, np.float32(c[0]), dtype=np.float32)
            for cj in c[1:]:
                acc = ((acc * x).astype(np.float64) + cj).astype(np.float32)
            s = np.cumsum(acc, dtype=np.float32)[-1]
        else:
            acc = np.full(n, c[0])
            for cj in c[1:]:
                acc = acc * x + cj
            s = np.cumsum(acc)[-1]
    assert np.array_equal(o["r"].view(np.uint8), acc.view(np.uint8))
    assert np.array_equal(np.array(o["s"]).reshape(1).view(np.uint8), np.array([s], dtype=dtype.np).view(np.uint8))
    if dtype is F32:
        # |x| >= 5 overflows single precision: +-inf rows, and the sum is NaN
        assert np.isinf(o["r"][0]) and np.isnan(o["s"])
    else:
        # the benchmark's `agree` check (bench.ml:157-164) against vanilla_poly
        assert abs(float(o["s"]) - RB.vanilla_poly_sum(c, x)) <= max(1e-3, abs(float(o["s"])) * 1e-3)


def test_refbench_saxpy_inputs():
    from cudacaml_amd.examples import refbench as RB

    n = 1 << 24
    x, y = RB.x_input(n), RB.y_input(n)
    # bench.ml:223-224: x[i] = (i mod 17) - 8, y[i] = (n - i) / 4, both exact in f32
    assert x[:18].tolist() == list(range(-8, 9)) + [-8]
    assert y[0] == n / 4 and y[-1] == 0.25 and float(y[12345]) == (n - 12345) / 4.0
    o = dict(run(RB.saxpy_graph(1000, F64), [("x", RB.x_input(1000, F64)), ("y", RB.y_input(1000, F64))]))
    xi = np.arange(1000) % 17 - 8.0
    assert o["r"].tolist() == (2.0 * xi + (1000 - np.arange(1000)) / 4.0).tolist()
