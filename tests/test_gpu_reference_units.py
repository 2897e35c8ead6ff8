"""The reference's unit-test graphs, run on the device.

test/unit/test_grad.ml, test_rows.ml, test_broadcast.ml, test_scatter.ml,
test_matmul.ml and test_black_scholes.ml check their graphs on the
interpreter. Here the same graphs run on Backend_hip: each case is
compared with the CPU oracle under the per-output policy (f64 to 1e-12,
integers bit for bit) and with the values the reference test itself
expects."""

import numpy as np
import pytest

from cudacaml_amd import dsl as D
from cudacaml_amd import grad as G
from cudacaml_amd.examples import black_scholes as bs
from cudacaml_amd.ir import F32, F64, I32, Graph

from test_gpu_parity import assert_policy

pytestmark = pytest.mark.gpu

Z = D.const(F64, 0.0)
XS4 = np.array([1.0, -2.0, 0.5, 3.0])
YS4 = np.array([0.3, 1.5, -1.0, 2.0])
M23 = np.array([[1.0, 2, 3], [4, 5, 6]])


def p64(name, dims):
    return D.param(name, F64, dims)


def one(name, t):
    return Graph.create("g", [(name, t)])


def s_of(t):
    return D.reduce(D.add, Z, t)


# (id, graph builder, inputs, output, wrt, {grad name: expected values})
GRAD_CASES = [
    ("sum_x2", lambda: one("s", s_of(D.map(lambda e: D.mul(e, e), p64("x", (4,))))),
     [("x", XS4)], "s", ["x"], {"ds/dx": 2 * XS4}),
    ("sum_xy", lambda: one("s", s_of(D.map2(D.mul, p64("x", (4,)), p64("y", (4,))))),
     [("x", XS4), ("y", YS4)], "s", ["x", "y"], {"ds/dx": YS4, "ds/dy": XS4}),
    ("chain", lambda: one("s", s_of(D.map2(lambda a, b: D.add(D.mul(D.exp(a), b), D.sin(D.mul(a, b))),
                                           p64("x", (4,)), p64("y", (4,))))),
     [("x", XS4), ("y", YS4)], "s", ["x", "y"], {}),
    ("reduce_max_argmax", lambda: one("m", D.reduce(D.max, D.const(F64, -1e300), p64("x", (4,)))),
     [("x", np.array([1.0, 5, 3, 2]))], "m", ["x"], {"dm/dx": [0, 1, 0, 0]}),
    ("reduce_rows_weights", lambda: one("s", s_of(D.map2(D.mul, p64("w", (2,)), D.reduce_rows(D.add, Z, p64("x", (2, 3)))))),
     [("x", M23), ("w", np.array([10.0, 20]))], "s", ["x", "w"], {"ds/dx": [[10, 10, 10], [20, 20, 20]]}),
    ("scan_reverse_cumsum", lambda: one("s", s_of(D.map2(D.mul, p64("w", (4,)), D.scan(D.add, Z, p64("x", (4,)))))),
     [("x", XS4), ("w", YS4)], "s", ["x"], {"ds/dx": [2.8, 2.5, 1.0, 2.0]}),
    ("scan_rows", lambda: one("s", s_of(D.map2(D.mul, p64("w", (2, 3)), D.scan_rows(D.add, Z, p64("x", (2, 3)))))),
     [("x", M23), ("w", M23)], "s", ["x"], {"ds/dx": [[6, 5, 3], [15, 11, 6]]}),
    ("broadcast", lambda: one("t", s_of(D.map2(D.mul, p64("x", (4,)), D.broadcast((4,), D.scalar("s", F64))))),
     [("x", XS4), ("s", np.array(1.7))], "t", ["s", "x"], {"dt/ds": XS4.sum(), "dt/dx": np.full(4, 1.7)}),
    ("reshape", lambda: one("s", s_of(D.map(lambda e: D.mul(e, e), D.reshape((6,), p64("x", (2, 3)))))),
     [("x", M23)], "s", ["x"], {"ds/dx": 2 * M23}),
    ("non_scalar_seed", lambda: one("r", D.map2(D.mul, p64("x", (4,)), p64("y", (4,)))),
     [("x", XS4), ("y", YS4)], "r", ["x"], {"dr/dx": YS4}),
    ("gather_repeated", lambda: one("s", s_of(D.gather(D.param("idx", I32, (3,)), p64("x", (3,))))),
     [("x", np.array([1.0, 2, 3])), ("idx", np.array([0, 0, 1], np.int32))], "s", ["x"], {"ds/dx": [2, 1, 0]}),
    ("gather_reverse", lambda: one("s", s_of(D.map2(D.mul, p64("w", (4,)), D.gather(
        D.map(lambda i: D.sub(D.const(I32, 3), i), D.iota((4,))), p64("x", (4,)))))),
     [("x", XS4), ("w", YS4)], "s", ["x"], {"ds/dx": YS4[::-1]}),
    ("matmul", lambda: one("s", s_of(D.matmul(p64("a", (2, 3)), p64("b", (3, 2))))),
     [("a", np.array([[1, -2, 0.5], [3, 1.5, -1]])), ("b", np.array([[0.3, 1.5], [-1, 2], [0.7, -0.2]]))],
     "s", ["a", "b"], {"ds/da": np.tile([1.8, 1.0, 0.5], (2, 1)), "ds/db": np.tile([[4.0], [-0.5], [-0.5]], (1, 2))}),
]


@pytest.mark.parametrize("name,graph,inputs,output,wrt,expect", GRAD_CASES, ids=[c[0] for c in GRAD_CASES])
def test_grad_rules_on_device(device, name, graph, inputs, output, wrt, expect):
    """test_grad.ml's graphs differentiated by Grad.grad and run on the
    device: every output within 1e-12 of the oracle, and the gradients the
    reference test states."""
    gg = G.grad(graph(), output, wrt)
    _, got = assert_policy(gg, inputs)
    o = dict(got)
    for k, v in expect.items():
        np.testing.assert_allclose(o[k], np.asarray(v, np.float64), rtol=0, atol=1e-9, err_msg=k)


def test_grad_unused_param_is_zeros_on_device(device):
    x, y = p64("x", (4,)), p64("y", (2, 2))
    g = Graph.create("g", [("s", s_of(x)), ("y", y)])
    _, got = assert_policy(G.grad(g, "s", ["y"]), [("x", XS4), ("y", YS4.reshape(2, 2))])
    assert dict(got)["ds/dy"].tolist() == [[0, 0], [0, 0]]


# ---- test_rows.ml, test_broadcast.ml ----------------------------------------


def rows_and_broadcast_cases():
    x23 = D.param("x", F32, (2, 3))
    yield "reduce_rows_add", Graph.create("g", [("r", D.reduce_rows(D.add, D.const(F32, 0.0), x23))]), \
        [("x", M23.astype(np.float32))], {"r": [6, 15]}
    yield "whole_tensor_reduce", Graph.create("g", [("s", D.reduce(D.add, D.const(F32, 0.0), D.param("x", F32, (2, 3))))]), \
        [("x", M23.astype(np.float32))], {"s": 21}
    xs = D.param("x", F32, (2, 3))
    yield "scan_rows_and_flat_scan", Graph.create("g", [
        ("r", D.scan_rows(D.add, D.const(F32, 0.0), xs)),
        ("f", D.scan(D.add, D.const(F32, 0.0), D.reshape((6,), xs)))]), \
        [("x", M23.astype(np.float32))], {"r": [[1, 3, 6], [4, 9, 15]], "f": [1, 3, 6, 10, 15, 21]}
    yield "reduce_rows_max", Graph.create("g", [("m", D.reduce_rows(D.max, D.const(F32, -1e30), D.param("x", F32, (2, 3))))]), \
        [("x", np.array([[3, -1, 2], [-5, -4, -6]], np.float32))], {"m": [3, -4]}
    yield "column_sums", Graph.create("g", [("c", D.reduce_rows(D.add, D.const(F32, 0.0), D.transpose(D.param("x", F32, (2, 3)))))]), \
        [("x", M23.astype(np.float32))], {"c": [5, 7, 9]}
    s = D.scalar("s", F32)
    yield "broadcast_scalar_param", Graph.create("g", [("r", D.broadcast((4,), s))]), \
        [("s", np.array(2.5, np.float32))], {"r": [2.5] * 4}
    x4 = D.param("x", F32, (4,))
    yield "x_times_broadcast_sum", Graph.create("g", [("r", D.map2(D.mul, x4, D.broadcast((4,), D.reduce(D.add, D.const(F32, 0.0), x4))))]), \
        [("x", np.array([1, 2, 3, 4], np.float32))], {"r": [10, 20, 30, 40]}
    yield "full_constant", Graph.create("g", [("c", D.full(F32, (2, 2), 7.0))]), [], {"c": [[7, 7], [7, 7]]}


@pytest.mark.parametrize("name,g,inputs,expect", list(rows_and_broadcast_cases()),
                         ids=[c[0] for c in rows_and_broadcast_cases()])
def test_rows_and_broadcast_on_device(device, name, g, inputs, expect):
    _, got = assert_policy(g, inputs)
    o = dict(got)
    for k, v in expect.items():
        np.testing.assert_array_equal(o[k], np.asarray(v, np.float32), err_msg=k)


# ---- test_scatter.ml, test_matmul.ml ----------------------------------------


def test_scatter_histograms_on_device(device):
    idx = np.array([0, 2, 2, 1, 2, 0, 3], np.int32)
    for dt, src in ((F32, np.array([0.5, 1, 2, 0.25, 3, 1.5, -1], np.float32)), (I32, np.arange(1, 8, dtype=np.int32))):
        g = Graph.create("h", [("h", D.scatter_add(D.param("i", I32, (7,)), D.param("x", dt, (7,)), (4,)))])
        _, got = assert_policy(g, [("i", idx), ("x", src)])
        want = np.zeros(4, src.dtype)
        np.add.at(want, idx, src)
        np.testing.assert_array_equal(dict(got)["h"], want)


def test_matmul_small_cases_on_device(device):
    a = D.param("a", F64, (2, 3))
    b = D.param("b", F64, (3, 2))
    _, got = assert_policy(Graph.create("m", [("c", D.matmul(a, b))]),
                           [("a", np.arange(1, 7, dtype=np.float64).reshape(2, 3)),
                            ("b", np.arange(7, 13, dtype=np.float64).reshape(3, 2))])
    assert dict(got)["c"].tolist() == [[58, 64], [139, 154]]
    eye = np.eye(4)
    m = np.arange(16, dtype=np.float64).reshape(4, 4)
    _, got = assert_policy(Graph.create("m", [("c", D.matmul(D.param("a", F64, (4, 4)), D.param("b", F64, (4, 4))))]),
                           [("a", eye), ("b", m)])
    np.testing.assert_array_equal(dict(got)["c"], m)
    av = np.array([((i * 7) % 11) - 5.0 for i in range(35)]).reshape(5, 7) / 3.0
    bv = np.array([((i * 5) % 13) / 4.0 for i in range(21)]).reshape(7, 3)
    _, got = assert_policy(Graph.create("m", [("c", D.matmul(D.param("a", F64, (5, 7)), D.param("b", F64, (7, 3))))]),
                           [("a", av), ("b", bv)])
    np.testing.assert_allclose(dict(got)["c"], av @ bv, rtol=0, atol=1e-12)


# ---- test_black_scholes.ml --------------------------------------------------


def test_black_scholes_mc_on_device(device):
    """call_mc at 65536 paths within 0.25 of the closed form, call_mc_paths
    16384 x 8 within 0.5; the Greeks graph's forward price equals call_mc's
    to the float64 band: the interpreter's two sums are the same sequence,
    the device's two fixed trees have different shapes (the Greeks graph
    folds its sum inside the kernel that writes the terminal prices)."""
    cf = bs.analytic()
    ins = bs.inputs(F64, seed=7)
    _, got = assert_policy(bs.call_mc(65536, F64), ins)
    price = bs.scalar_out(got, "price")
    assert abs(price - cf["price"]) <= 0.25
    _, got = assert_policy(bs.call_mc_paths(16384, 8, F64), ins)
    assert abs(bs.scalar_out(got, "price") - cf["price"]) <= 0.5
    _, got = assert_policy(bs.call_greeks(65536, F64), ins)
    assert abs(bs.scalar_out(got, "price") - price) <= 1e-12 * (1 + abs(price))
