"""Differential's contract, pinned with fake backends that wrap the oracle
(test/unit/test_executor.ml:20-73): a 0.1 % error fails at the default
tolerance and names the output, passes at 1e-2; output order is free; a
missing output and a raising backend are errors, not exceptions. Plus the
per-output policy bar. No GPU."""

import numpy as np

import oracle
from cudacaml_amd import differential as Diff
from cudacaml_amd import dsl as D
from cudacaml_amd.examples import programs as P
from cudacaml_amd.ir import F32, I32, Graph


def corrupt(outs):
    (n, v), rest = outs[0], outs[1:]
    v = v.copy()
    flat = v.reshape(-1)
    if v.dtype.kind == "f":
        flat[1] = flat[1] * 1.001
    else:
        flat[1] = np.iinfo(v.dtype).max
    return [(n, v)] + rest


class Slight:
    name = "slight"
    compile = staticmethod(oracle.Interp.compile)

    @staticmethod
    def run(c, inputs):
        return corrupt(oracle.Interp.run(c, inputs))


class Reordered:
    name = "reordered"
    compile = staticmethod(oracle.Interp.compile)

    @staticmethod
    def run(c, inputs):
        return list(reversed(oracle.Interp.run(c, inputs)))


class Missing:
    name = "missing"
    compile = staticmethod(oracle.Interp.compile)

    @staticmethod
    def run(c, inputs):
        return oracle.Interp.run(c, inputs)[1:]


class Boom:
    name = "boom"

    @staticmethod
    def compile(g):
        return None

    @staticmethod
    def run(c, inputs):
        raise RuntimeError("boom")


def check(cand, e, tol=1e-5):
    return Diff.check(oracle.Interp, cand, e.graph(), e.inputs(), tolerance=tol)


def test_interp_agrees_with_itself():
    for e in P.all_examples():
        assert check(oracle.Interp, e) == (True, None)


def test_contract():
    ok, msg = check(Slight, P.saxpy(16))
    assert not ok and "r" in msg
    assert check(Slight, P.saxpy(16), tol=1e-2) == (True, None)
    assert check(Reordered, P.saxpy(16)) == (True, None)
    assert check(Missing, P.saxpy(16))[0] is False
    ok, msg = check(Boom, P.saxpy(16))
    assert not ok and "boom" in msg


def test_nan_equals_nan_and_dtype_shape_mismatch():
    e = [("a", np.array([np.nan, 1.0], np.float32))]
    assert Diff.compare_all(e, [("a", np.array([np.nan, 1.0], np.float32))]) == (True, None)
    assert Diff.compare_all(e, [("a", np.array([np.nan, 1.0], np.float64))])[0] is False
    assert Diff.compare_all(e, [("a", np.array([np.nan], np.float32))])[0] is False


def test_ulp_distance():
    a = np.array([1.0, -1.0, 0.0, np.nan], np.float32)
    b = np.nextafter(a, np.float32(np.inf))
    assert Diff.ulp_distance_f32(a, b).tolist()[:3] == [1, 1, 1]
    assert Diff.ulp_distance_f32(np.float32(0.0), np.float32(-0.0)) == 0
    assert Diff.ulp_distance_f32(np.array([np.nan], np.float32), np.array([np.nan], np.float32)).tolist() == [0]


def test_policy_rules():
    x = D.param("x", F32, (4,))
    i = D.param("i", I32, (4,))
    g = Graph.create("g", [("m", D.map(D.exp, x)), ("s", D.reduce(D.add, D.const(F32, 0.0), x)),
                           ("k", D.map(lambda e: D.add(e, e), i))])
    rules = {n: Diff.rule_for(t) for n, t in g.outputs}
    assert rules == {"m": "ulp2", "s": "rel1e-4", "k": "exact"}
    e = [("m", np.float32([1, 2, 3, 4])), ("s", np.float32(10.0)), ("k", np.int32([1, 2, 3, 4]))]
    got = [("m", np.nextafter(np.float32([1, 2, 3, 4]), np.float32(9))), ("s", np.float32(10.0005)),
           ("k", np.int32([1, 2, 3, 4]))]
    vs = {v.name: v for v in Diff.policy_check(g, e, got)}
    assert vs["m"].ok and vs["s"].ok and vs["k"].ok
    got[2] = ("k", np.int32([1, 2, 3, 5]))
    assert not {v.name: v for v in Diff.policy_check(g, e, got)}["k"].ok
