"""The reference benchmark's workloads (bench/bench.ml:1-300).

``cudacaml-bench`` times two graphs as whole runs (upload, launch,
download), best of ``reps``, and prints GFLOP/s for the second:

* saxpy at a chosen dtype: ``r = a*x + y``, ``s = sum r``, a = 2
  (``saxpy_graph``, bench.ml:118-126);
* poly, a Horner recurrence of ``degree`` coefficients built as
  ``degree - 1`` chained maps, plus ``s = sum r`` (``poly_graph``,
  bench.ml:97-111). Fusion collapses the chain into one kernel, so the
  plan is two kernels whatever the degree. It does ``2*degree - 1`` flops
  per element (bench.ml:254).

Inputs are the benchmark's own: ``x[i] = (i mod 17) - 8``,
``y[i] = (n - i) / 4`` (bench.ml:223-224), and coefficients
``c[j] = 1 / (j + 1)`` (bench.ml:253). Published results
(bench/results/nvidia-a100-sxm4-40gb.md:36-37) are quoted with them.
"""

from __future__ import annotations

import numpy as np

from .. import dsl as D
from ..ir import F32, Graph

DEGREE = 64
N = 1 << 24

# bench/results/nvidia-a100-sxm4-40gb.md:36-37, n = 2^24, best of 5 whole runs
PUBLISHED_A100 = {
    "f32": {"saxpy_cuda_s": 0.09306, "poly_cuda_s": 0.07816, "poly_gflops": 27.26},
    "f64": {"saxpy_cuda_s": 0.1714, "poly_cuda_s": 0.1446, "poly_gflops": 14.73},
}


def coefficients(degree=DEGREE):
    """``c[j] = 1 / (j + 1)`` as OCaml floats (bench.ml:253)."""
    return [1.0 / float(j + 1) for j in range(degree)]


def poly_flops(degree=DEGREE):
    return 2 * degree - 1


def poly_graph(n=N, dtype=F32, c=None):
    """``acc_0 = c0`` (a map of x to the constant), then
    ``acc_j = acc_{j-1} * x + c_j`` as one map2 per coefficient;
    outputs ``r = acc`` and ``s = reduce add 0 acc`` (bench.ml:101-111)."""
    c = coefficients() if c is None else list(c)
    if not c:
        raise ValueError("poly_graph: no coefficients")
    x = D.param("x", dtype, (n,))
    acc = D.map(lambda _e, c0=c[0]: D.const(dtype, c0), x)
    for ci in c[1:]:
        acc = D.map2(lambda a, xi, ci=ci: D.add(D.mul(a, xi), D.const(dtype, ci)), acc, x)
    return Graph.create("poly", [("r", acc), ("s", D.reduce(D.add, D.const(dtype, 0.0), acc))])


def saxpy_graph(n=N, dtype=F32, a=2.0):
    """The shape of ``Saxpy.program`` at a chosen dtype (bench.ml:118-126)."""
    x = D.param("x", dtype, (n,))
    y = D.param("y", dtype, (n,))
    r = D.map2(D.add, D.map(lambda xi: D.mul(D.const(dtype, a), xi), x), y)
    return Graph.create("saxpy", [("r", r), ("s", D.reduce(D.add, D.const(dtype, 0.0), r))])


def x_input(n=N, dtype=F32):
    return (np.arange(n, dtype=np.int64) % 17 - 8).astype(dtype.np)


def y_input(n=N, dtype=F32):
    return ((n - np.arange(n, dtype=np.int64)) / 4.0).astype(dtype.np)


def vanilla_poly_sum(c, x):
    """``vanilla_poly`` (bench.ml:70-82): the Horner loop over doubles, its
    running sum of r. Only the sum is returned, as the benchmark's
    ``agree`` check uses it."""
    acc = np.full(x.shape, c[0], dtype=np.float64)
    xd = x.astype(np.float64)
    for cj in c[1:]:
        acc = acc * xd + cj
    return float(np.sum(acc))
