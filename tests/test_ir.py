"""The front end the backend serves: Dsl shape checks, Graph.create
(topological order, uses-based fan-out, params, errors), the wire format
and its two parsers (the oracle's and the backend's must agree).
Restates test_graph.ml / test_rows.ml:81-86 / test_scatter.ml:47-49 /
test_matmul.ml:101-104. No GPU."""

import numpy as np
import pytest

import oracle
from cudacaml_amd import backend_hip as H
from cudacaml_amd import dsl as D
from cudacaml_amd import ir
from cudacaml_amd.examples import black_scholes as bs
from cudacaml_amd.examples import programs as P
from cudacaml_amd.ir import F32, F64, I32, Graph


def test_shape_checks_raise():
    v = D.param("v", F32, (5,))
    r3 = D.param("w", F32, (2, 2, 2))
    z = D.const(F32, 0.0)
    for f in (lambda: D.reduce_rows(D.add, z, v), lambda: D.scan_rows(D.add, z, v),
              lambda: D.transpose(v), lambda: D.transpose(r3)):
        with pytest.raises(ValueError):
            f()
    with pytest.raises(ValueError, match="shape mismatch"):
        D.map2(D.add, v, D.param("u", F32, (4,)))
    with pytest.raises(ValueError, match="numel mismatch"):
        D.reshape((4,), v)
    with pytest.raises(ValueError, match="exactly one element"):
        D.broadcast((3,), v)
    with pytest.raises(ValueError):
        D.scatter_add(D.param("i", I32, (6,)), D.param("s", F32, (5,)), (4,))
    with pytest.raises(ValueError, match="cannot be accumulated"):
        D.scatter_add(D.param("i", I32, (6,)), D.param("s", ir.I64, (6,)), (4,))
    for a, b in [((2, 3), (2, 3)), ((6,), (6,)), ((2, 2, 2), (2, 2))]:
        with pytest.raises(ValueError, match="Dsl.matmul"):
            D.matmul(D.param("a", F64, a), D.param("b", F64, b))


def test_reduce_shapes():
    x = D.param("x", F32, (2, 3, 4))
    z = D.const(F32, 0.0)
    assert D.reduce_rows(D.add, z, x).shape == (2, 3)
    assert D.reduce(D.add, z, x).shape == ()
    assert D.scan(D.add, z, x).shape == (2, 3, 4)


def test_graph_create_errors():
    x = D.param("x", F32, (2,))
    with pytest.raises(ValueError, match="at least one output"):
        Graph.create("g", [])
    with pytest.raises(ValueError, match="duplicate output"):
        Graph.create("g", [("a", x), ("a", D.map(D.neg, x))])
    y = D.param("x", F32, (2,))
    with pytest.raises(ValueError, match="two Param nodes"):
        Graph.create("g", [("a", D.map2(D.add, x, y))])


def test_topological_order_and_fan_out():
    x = D.param("x", F32, (4,))
    s = D.map(lambda e: D.mul(e, e), x)
    a = D.map2(D.add, s, s)
    g = Graph.create("g", [("a", a), ("s", s)])
    order = [t.uid for t in g.order]
    assert order.index(x.uid) < order.index(s.uid) < order.index(a.uid)
    # uses, not consumers: map2 add s s counts 2; outputs are not uses
    assert g.fan_out_of(s) == 2 and g.fan_out_of(a) == 0 and g.fan_out_of(x) == 1
    assert [n for n, _ in g.params] == ["x"]
    assert "Map2" in g.to_dot()


def test_deep_chain_has_no_recursion_limit():
    x = D.param("x", F32, (4,))
    t = x
    for _ in range(5000):
        t = D.map(D.neg, t)
    g = Graph.create("deep", [("r", t)])
    assert len(g.order) == 5001


def test_wire_round_trip_through_both_parsers():
    """Every example's wire text is accepted by the oracle and by the
    backend's parser, and the backend reports the same params/outputs."""
    for e in P.all_examples():
        g = e.graph()
        w = g.to_wire()
        assert w.startswith("cchip-graph 1 ") and w.rstrip().endswith("end")
        oracle.Interp.compile(g)
        plan = H.plan(g)
        assert plan.startswith("program ")
        outs = [l.split()[1] for l in plan.splitlines() if l.startswith("download")]
        assert outs == [n for n, _ in g.outputs]


def test_wire_names_are_escaped():
    x = D.param("x y%", F32, (2,))
    g = Graph.create("na me", [("out put", D.map(D.neg, x))])
    o = oracle.run(g, [("x y%", np.array([1, 2], np.float32))])
    assert o[0][0] == "out put" and o[0][1].tolist() == [-1, -2]
    assert "upload x y% p_x y%" in H.plan(g) or "x%20y%25" not in H.plan(g)


def test_shared_expressions_are_written_once():
    from cudacaml_amd import rng

    g = Graph.create("u", [("r", rng.u32(D.scalar("seed", I32), (8,)))])
    lines = g.to_wire().splitlines()
    # Philox-10 is a DAG of a few hundred nodes, not an exponential tree.
    assert len([l for l in lines if l.startswith("x ")]) < 400


def test_malformed_wire_is_rejected():
    bad = "cchip-graph 1 g\nt 1 map f32 1 2 99 98\no r 1\nend\n"
    with pytest.raises(ValueError, match="unknown"):
        from cudacaml_amd._lib import check, lib
        import ctypes

        out = ctypes.c_void_p()
        check(lib().cchip_backend_plan(bad.encode(), ctypes.byref(out)))
    with pytest.raises(oracle.OracleError):
        import ctypes

        lib_o = oracle._load()
        err = ctypes.create_string_buffer(256)
        h = lib_o.orc_parse(bad.encode(), err, 256)
        if not h:
            raise oracle.OracleError(err.value.decode())


def test_greeks_graph_structure():
    g = bs.call_greeks(4096, F64)
    assert sorted(n for n, _ in g.params) == ["rate", "s0", "seed", "vol"]
    assert [n for n, _ in g.outputs] == ["price", "dprice/ds0", "dprice/dvol", "dprice/drate"]
    kernels = [l for l in H.plan(g).splitlines() if l.startswith("kernel")]
    assert len(kernels) < 40


@pytest.mark.parametrize("dims", ["2 4294967296 4294967296", "2 65536 65536", "1 2147483648", "2 0 2147483648",
                                  "3 2048 2048 512"])
def test_wire_extents_that_wrap_or_exceed_2_31_are_rejected(dims):
    """Element counts are checked before each multiplication: [2^32; 2^32]
    (whose 64-bit product wraps to 0) and every tensor of 2^31 elements or
    more, or with such an extent, is rejected by the backend's parser."""
    import ctypes

    from cudacaml_amd._lib import check, lib

    wire = "cchip-graph 1 g\nt 1 param f32 %s x\no r 1\nend\n" % dims
    out = ctypes.c_void_p()
    with pytest.raises(ValueError, match="2\\^31-1 elements"):
        check(lib().cchip_backend_plan(wire.encode(), ctypes.byref(out)))
    lib_o = oracle._load()
    err = ctypes.create_string_buffer(256)
    if dims.startswith("2 4294967296"):
        assert not lib_o.orc_parse(wire.encode(), err, 256)
        assert b"too many elements" in err.value


def test_wire_largest_tensor_is_accepted():
    import ctypes

    from cudacaml_amd._lib import check, lib

    wire = "cchip-graph 1 g\nt 1 param i32 2 32767 65537 x\no r 1\nend\n"
    out = ctypes.c_void_p()
    check(lib().cchip_backend_plan(wire.encode(), ctypes.byref(out)))
    lib().cchip_free(out)
