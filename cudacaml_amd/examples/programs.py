"""Registry of example programs with deterministic inputs
(examples/programs.ml:16-148): every input is a closed-form formula."""

from __future__ import annotations

import numpy as np

from .. import dsl as D
from ..ir import F32, F64, I32, Graph
from . import black_scholes as bs
from . import saxpy as sx


class Example:
    __slots__ = ("name", "graph", "inputs")

    def __init__(self, name, graph, inputs):
        self.name = name
        self.graph = graph
        self.inputs = inputs


def f32s(shape, f):
    n = int(np.prod(shape)) if len(shape) else 1
    return np.array([f(i) for i in range(n)], dtype=np.float32).reshape(shape)


def x_in(n):
    return ("x", (np.arange(n) % 17 - 8).astype(np.float32))


def y_in(n):
    return ("y", ((n - np.arange(n)) / 4.0).astype(np.float32))


def saxpy(n):
    return Example("saxpy", lambda: sx.program(n, 2.0), lambda: [x_in(n), y_in(n)])


def sum_(n):
    def graph():
        x = D.param("x", F32, (n,))
        return Graph.create("sum", [("s", D.reduce(D.add, D.const(F32, 0.0), x))])
    return Example("sum", graph, lambda: [x_in(n)])


def maxval(n):
    def graph():
        x = D.param("x", F32, (n,))
        return Graph.create("maxval", [("m", D.reduce(D.max, D.const(F32, -1e30), x))])
    return Example("maxval", graph, lambda: [x_in(n)])


def prefix(n):
    def graph():
        x = D.param("x", F32, (n,))
        return Graph.create("prefix", [("p", D.scan(D.add, D.const(F32, 0.0), x))])
    return Example("prefix", graph, lambda: [x_in(n)])


def reverse(n):
    def graph():
        x = D.param("x", F32, (n,))
        idx = D.map(lambda i: D.sub(D.const(I32, n - 1), i), D.iota((n,)))
        return Graph.create("reverse", [("r", D.gather(idx, x))])
    return Example("reverse", graph, lambda: [x_in(n)])


def clamp(n):
    def graph():
        x = D.param("x", F32, (n,))
        zero, one = D.const(F32, 0.0), D.const(F32, 1.0)
        r = D.map(lambda e: D.select(D.lt(e, zero), zero, D.select(D.lt(one, e), one, e)), x)
        return Graph.create("clamp", [("r", r)])
    return Example("clamp", graph, lambda: [x_in(n)])


def squares(n):
    def graph():
        def f(i):
            fi = D.cast(F32, i)
            return D.mul(fi, fi)
        return Graph.create("squares", [("r", D.map(f, D.iota((n,))))])
    return Example("squares", graph, lambda: [])


def chain(n):
    """Five chained maps: one kernel."""
    def graph():
        x = D.param("x", F32, (n,))
        one = D.const(F32, 1.0)
        r = D.map(lambda e: D.add(e, one), x)
        r = D.map(lambda e: D.mul(e, e), r)
        r = D.map(D.neg, r)
        r = D.map(lambda e: D.sub(e, one), r)
        r = D.map(lambda e: D.mul(e, D.const(F32, 0.5)), r)
        return Graph.create("chain", [("r", r)])
    return Example("chain", graph, lambda: [x_in(n)])


def fanout(n):
    def graph():
        x = D.param("x", F32, (n,))
        s = D.map(lambda e: D.mul(e, e), x)
        return Graph.create("fanout", [("a", D.map(D.neg, s)), ("b", D.map(D.sqrt, s)),
                                       ("c", D.reduce(D.add, D.const(F32, 0.0), s))])
    return Example("fanout", graph, lambda: [x_in(n)])


def reshape_flat():
    def graph():
        x = D.param("x", F32, (4, 8))
        return Graph.create("reshape_flat", [("r", D.map(D.neg, D.reshape((32,), x)))])
    return Example("reshape_flat", graph, lambda: [("x", np.arange(32, dtype=np.float32).reshape(4, 8))])


bs_dtype = F64
bs_seed = 7


def bs_mc(n_paths):
    return Example("bs_mc", lambda: bs.call_mc(n_paths, bs_dtype), lambda: bs.inputs(bs_dtype, seed=bs_seed))


def bs_paths(n_paths, n_steps):
    return Example("bs_paths", lambda: bs.call_mc_paths(n_paths, n_steps, bs_dtype),
                   lambda: bs.inputs(bs_dtype, seed=bs_seed))


def bs_greeks(n_paths):
    return Example("bs_greeks", lambda: bs.call_greeks(n_paths, bs_dtype), lambda: bs.inputs(bs_dtype, seed=bs_seed))


def all_examples():
    return [saxpy(1024), sum_(1000), maxval(257), prefix(300), reverse(100), clamp(512), squares(64),
            chain(4096), fanout(1000), reshape_flat(), bs_mc(4096), bs_paths(512, 16), bs_greeks(4096)]


def find(name):
    for e in all_examples():
        if e.name == name:
            return e
    return None
