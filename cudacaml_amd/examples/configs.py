"""The five benchmark configurations and their synthetic inputs.

Inputs come from the same generator as ``Rng.u32``:
``G(seed, i) = philox4x32_10((i, 0, 0, 0), (seed, 0)).w0``. Formulas:

* uniform in [-1, 1), exactly representable: ``((G >> 8) - 2^23) * 2^-23``
* small integers in [0, 16): ``G >> 28``
* bin indices in [0, 2^20): ``G >> 12``
* N(0, 1): ``sqrt 2 * erfinv(2u - 1)`` with ``u = (G + 0.5) 2^-32``, in f64
  then cast (``Rng.normal_inv_cdf``)
* a permutation of [0, n): the argsort of ``G``, ties by index

Every input exists twice: a numpy generator (tests, the CPU baseline) and
a graph that computes it on the device (the benchmark, so 2^28-element
inputs are not generated on the host).
"""

from __future__ import annotations

import math

import numpy as np

from .. import dsl as D
from .. import grad as G
from .. import rng
from ..ir import F32, F64, I32, Graph
from . import black_scholes as bs
from . import programs as P
from . import saxpy as sx

M0, M1, W0, W1 = 0xD2511F53, 0xCD9E8D57, 0x9E3779B9, 0xBB67AE85


def philox_w0(seed, n, start=0, chunk=1 << 22):
    """Word 0 of Philox-4x32-10 at counters start..start+n-1, key (seed, 0),
    vectorised over uint64 lanes."""
    out = np.empty(n, dtype=np.uint32)
    mask = np.uint64(0xFFFFFFFF)
    for lo in range(0, n, chunk):
        hi = min(n, lo + chunk)
        c0 = np.arange(start + lo, start + hi, dtype=np.uint64) & mask
        c1 = np.zeros_like(c0)
        c2 = np.zeros_like(c0)
        c3 = np.zeros_like(c0)
        k0 = np.uint64(seed & 0xFFFFFFFF)
        k1 = np.uint64(0)
        for r in range(10):
            p0 = np.uint64(M0) * c0
            p1 = np.uint64(M1) * c2
            n0 = (p1 >> np.uint64(32)) ^ c1 ^ k0
            n1 = p1 & mask
            n2 = (p0 >> np.uint64(32)) ^ c3 ^ k1
            n3 = p0 & mask
            c0, c1, c2, c3 = n0, n1, n2, n3
            k0 = (k0 + np.uint64(W0)) & mask
            k1 = (k1 + np.uint64(W1)) & mask
        out[lo:hi] = c0.astype(np.uint32)
    return out


def uniform_pm1(seed, shape):
    n = int(np.prod(shape)) if len(shape) else 1
    w = philox_w0(seed, n)
    return (((w >> 8).astype(np.int64) - (1 << 23)).astype(np.float32) * np.float32(2.0 ** -23)).reshape(shape)


def small_ints(seed, shape):
    n = int(np.prod(shape))
    return (philox_w0(seed, n) >> 28).astype(np.int32).reshape(shape)


def bin_indices(seed, n, bits=20):
    return (philox_w0(seed, n) >> (32 - bits)).astype(np.int32)


def normals(seed, shape, dtype=F32):
    from scipy.special import erfinv

    n = int(np.prod(shape))
    u = (philox_w0(seed, n).astype(np.float64) + 0.5) * 2.3283064365386963e-10
    z = math.sqrt(2.0) * erfinv(2.0 * u - 1.0)
    return z.astype(dtype.np).reshape(shape)


def permutation(seed, n):
    return np.argsort(philox_w0(seed, n), kind="stable").astype(np.int32)


# ---------------------------------------------------------------------------
# Device-side generators: graphs whose one output is the input tensor.
# ---------------------------------------------------------------------------


def _u32(shape):
    return rng.u32(D.scalar("seed", I32), shape)


def gen_uniform_pm1(shape):
    def f(w):
        top = D.shr(w, D.const(I32, 8))
        return D.mul(D.cast(F32, D.sub(top, D.const(I32, 1 << 23))), D.const(F32, 2.0 ** -23))
    return Graph.create("gen_uniform", [("v", D.map(f, _u32(shape)))])


def gen_small_ints(shape):
    return Graph.create("gen_ints", [("v", D.map(lambda w: D.shr(w, D.const(I32, 28)), _u32(shape)))])


def gen_bin_indices(n, bits=20):
    return Graph.create("gen_bins", [("v", D.map(lambda w: D.shr(w, D.const(I32, 32 - bits)), _u32((n,))))])


def gen_normals(shape, dtype=F32):
    def f(w):
        return D.cast(dtype, rng.normal_inv_cdf(D.cast(F64, rng.to_unit_interval(F64, w))))
    return Graph.create("gen_normals", [("v", D.map(f, _u32(shape)))])


# ---------------------------------------------------------------------------
# Config graphs
# ---------------------------------------------------------------------------

N1 = 1 << 24
ROWS2 = 8192
SCAN2 = 1 << 28
N3 = 1 << 26
BINS3 = 1 << 20
MM_F32 = 4096
MM_F64 = 2048
PATHS5 = 1 << 22
STEPS5 = 64


def saxpy(n=N1):
    return sx.program(n, 2.0)


def chain(n=N1):
    return P.chain(n).graph()


def rows(r=ROWS2, c=ROWS2, dtype=F32):
    """reduce_rows add, reduce_rows max and scan_rows add over one matrix."""
    x = D.param("x", dtype, (r, c))
    z = D.const(dtype, 0.0)
    return Graph.create("rows", [
        ("sum", D.reduce_rows(D.add, z, x)),
        ("max", D.reduce_rows(D.max, D.const(dtype, -math.inf), x)),
        ("scan", D.scan_rows(D.add, z, x)),
    ])


def global_scan(n=SCAN2):
    v = D.param("v", I32, (n,))
    return Graph.create("global_scan", [("p", D.scan(D.add, D.const(I32, 0), v))])


def scatter_gather(n=N3, bins=BINS3, dtype=F32):
    idx = D.param("idx", I32, (n,))
    src = D.param("src", dtype, (n,))
    h = D.scatter_add(idx, src, (bins,))
    return Graph.create("scatter_gather", [("h", h), ("back", D.gather(idx, h))])


def matmul(n=MM_F32, dtype=F32, k=None, m=None):
    m = n if m is None else m
    k = n if k is None else k
    a = D.param("a", dtype, (m, k))
    b = D.param("b", dtype, (k, n))
    return Graph.create("matmul", [("c", D.matmul(a, b))])


def matmul_grad(n=MM_F32, dtype=F32):
    """Adjoint of sum(A@B) w.r.t. A and B: two more matmuls over transposes."""
    a = D.param("a", dtype, (n, n))
    b = D.param("b", dtype, (n, n))
    s = D.reduce(D.add, D.const(dtype, 0.0), D.matmul(a, b))
    return G.grad(Graph.create("mm", [("s", s)]), "s", ["a", "b"])


def mc_paths(n_paths=PATHS5, n_steps=STEPS5, dtype=F32):
    return bs.call_mc_paths(n_paths, n_steps, dtype)


def mc_greeks(n_paths=PATHS5, n_steps=STEPS5, dtype=F32):
    return bs.call_paths_greeks(n_paths, n_steps, dtype)
