"""saxpy: ``r = a*x + y`` then ``s = sum r`` (examples/saxpy.ml:10-17)."""

from __future__ import annotations

from .. import dsl as D
from ..ir import F32, Graph


def program(n, a, dtype=F32):
    shape = (n,)
    x = D.param("x", dtype, shape)
    y = D.param("y", dtype, shape)
    ax = D.map(lambda xi: D.mul(D.const(dtype, a), xi), x)
    r = D.map2(D.add, ax, y)
    s = D.reduce(D.add, D.const(dtype, 0.0), r)
    return Graph.create("saxpy", [("r", r), ("s", s)])
