"""Longstaff-Schwartz: an American put by least-squares Monte Carlo
(examples/lsm.ml).

Paths are simulated once (normal draws and a ``scan_rows`` of the
log-increments, as in ``black_scholes.call_mc_paths``). The algorithm then
walks backwards through the exercise dates. At each date the discounted
continuation value is regressed on the basis [1; S/K; (S/K)^2] over the
in-the-money paths, through the normal equations: two matmuls per step,
``X^T X : [3;3]`` and ``X^T y : [3;1]``, then a 3x3 solve on the host.
Everything is F64.

Three graphs are compiled once and only run afterwards; the time index
``t`` and the coefficients ``beta`` are params, so the loop never rebuilds
or re-JITs anything (lsm.ml:14-18).
"""

from __future__ import annotations

import math

import numpy as np

from .. import dsl as D
from .. import rng
from ..ir import F64, I32, Graph
from .black_scholes import analytic, market

DT = F64


# --------------------------------------------------------------------------
# Host-side references (lsm.ml:27-66)
# --------------------------------------------------------------------------


def binomial_american_put(steps, m=market):
    """Cox-Ross-Rubinstein binomial American put (lsm.ml:34-52)."""
    dt = m.maturity / steps
    u = math.exp(m.vol * math.sqrt(dt))
    d = 1.0 / u
    disc = math.exp(-m.rate * dt)
    p = ((1.0 / disc) - d) / (u - d)
    j = np.arange(steps + 1, dtype=np.float64)
    v = np.maximum(m.strike - m.s0 * u ** j * d ** (steps - j), 0.0)
    for i in range(steps - 1, -1, -1):
        jj = j[: i + 1]
        cont = disc * (p * v[1: i + 2] + (1.0 - p) * v[: i + 1])
        v = np.maximum(cont, m.strike - m.s0 * u ** jj * d ** (i - jj))
    return float(v[0])


def european_put(m=market):
    """Put-call parity on the analytic call (lsm.ml:58-60)."""
    return analytic(m)["price"] - m.s0 + m.strike * math.exp(-m.rate * m.maturity)


def solve3(a0, b0):
    """Gaussian elimination with partial pivoting; a singular or non-finite
    system yields zeros, meaning no early exercise at this date
    (lsm.ml:71-108)."""
    a = [list(map(float, r)) for r in a0]
    b = [float(v) for v in b0]
    x = [0.0, 0.0, 0.0]
    try:
        for k in range(3):
            piv = k
            for i in range(k + 1, 3):
                if abs(a[i][k]) > abs(a[piv][k]):
                    piv = i
            if not abs(a[piv][k]) > 1e-300:
                raise ArithmeticError
            if piv != k:
                a[k], a[piv] = a[piv], a[k]
                b[k], b[piv] = b[piv], b[k]
            for i in range(k + 1, 3):
                f = a[i][k] / a[k][k]
                for j in range(k, 3):
                    a[i][j] = a[i][j] - f * a[k][j]
                b[i] = b[i] - f * b[k]
        for i in range(2, -1, -1):
            s = b[i]
            for j in range(i + 1, 3):
                s = s - a[i][j] * x[j]
            x[i] = s / a[i][i]
        if not all(math.isfinite(v) for v in x):
            raise ArithmeticError
    except (ArithmeticError, ZeroDivisionError):
        x = [0.0, 0.0, 0.0]
    return x


# --------------------------------------------------------------------------
# The graphs (lsm.ml:118-240)
# --------------------------------------------------------------------------


def _kf(v):
    return D.const(DT, v)


def _ki(v):
    return D.const(I32, v)


def paths_graph(n_paths, n_steps, m=market):
    """``S : [n_paths; n_steps]``, column t at time (t+1) dt; exact GBM, the
    only param is the seed (lsm.ml:129-150)."""
    grid = (n_paths, n_steps)
    seed = D.scalar("seed", I32)
    dt = m.maturity / n_steps
    drift = (m.rate - 0.5 * m.vol * m.vol) * dt
    vol_dt = m.vol * math.sqrt(dt)
    z = rng.normal(DT, seed, grid)
    incr = D.map(lambda zi: D.add(_kf(drift), D.mul(_kf(vol_dt), zi)), z)
    cum = D.scan_rows(D.add, _kf(0.0), incr)
    s = D.map(lambda c: D.mul(_kf(m.s0), D.exp(c)), cum)
    return Graph.create("lsm_paths", [("S", s)])


def _basis(n_paths, n_steps, strike):
    """Column t of S by gather, the in-the-money mask, and the masked design
    matrix built from ``iota [n_paths; 3]`` (lsm.ml:168-191)."""
    grid = (n_paths, n_steps)
    g3 = (n_paths, 3)
    s = D.param("S", DT, grid)
    cf = D.param("cf", DT, (n_paths,))
    tb = D.broadcast((n_paths,), D.scalar("t", I32))
    idx = D.map2(lambda p, tv: D.add(D.mul(p, _ki(n_steps)), tv), D.iota((n_paths,)), tb)
    st = D.gather(idx, s)
    itm = D.map(lambda x: D.select(D.lt(x, _kf(strike)), _kf(1.0), _kf(0.0)), st)
    row = D.map(lambda k: D.div(k, _ki(3)), D.iota(g3))
    st3 = D.gather(row, st)
    itm3 = D.gather(row, itm)

    def phi_f(k, sv):
        j = D.sub(k, D.mul(D.div(k, _ki(3)), _ki(3)))
        x = D.div(sv, _kf(strike))
        return D.select(D.eq(j, _ki(0)), _kf(1.0), D.select(D.eq(j, _ki(1)), x, D.mul(x, x)))

    phi = D.map2(phi_f, D.iota(g3), st3)
    return cf, st, itm, D.map2(D.mul, phi, itm3)


def regress_graph(n_paths, n_steps, strike, disc):
    """The normal equations: ``xtx = X^T X`` and ``xty = X^T y`` with y the
    masked cash flow discounted one step (lsm.ml:199-210)."""
    cf, _, itm, xm = _basis(n_paths, n_steps, strike)
    y = D.map2(lambda c, mk: D.mul(D.mul(_kf(disc), c), mk), cf, itm)
    xt = D.transpose(xm)
    return Graph.create("lsm_regress", [("xtx", D.matmul(xt, xm)),
                                        ("xty", D.matmul(xt, D.reshape((n_paths, 1), y)))])


def update_graph(n_paths, n_steps, strike, disc):
    """The exercise decision: exercise where the intrinsic value is positive
    and beats the fitted continuation, otherwise keep the discounted
    realised cash flow (lsm.ml:217-236)."""
    cf, st, _, xm = _basis(n_paths, n_steps, strike)
    beta = D.param("beta", DT, (3, 1))
    cont = D.reshape((n_paths,), D.matmul(xm, beta))

    def exercises(s, c):
        e = D.max(D.sub(_kf(strike), s), _kf(0.0))
        return D.and_(D.gt(e, _kf(0.0)), D.gt(e, c))

    exv = D.map2(lambda s, c: D.select(exercises(s, c), D.sub(_kf(strike), s), _kf(0.0)), st, cont)
    keep = D.map2(lambda s, c: D.select(exercises(s, c), _kf(0.0), _kf(1.0)), st, cont)
    held = D.map2(lambda k, c: D.mul(k, D.mul(_kf(disc), c)), keep, cf)
    return Graph.create("lsm_update", [("cf", D.map2(D.add, exv, held))])


def _beta(xtx, xty):
    """Below three in-the-money paths the fit is not determined and the
    regression is skipped (lsm.ml:295-305)."""
    xtx = np.asarray(xtx, np.float64).reshape(-1)
    if xtx[0] < 3.0:
        return np.zeros((3, 1))
    a = [[xtx[i * 3 + j] + (1e-10 if i == j else 0.0) for j in range(3)] for i in range(3)]
    return np.array(solve3(a, np.asarray(xty, np.float64).reshape(-1)), np.float64).reshape(3, 1)


def _scalar_i32(v):
    return np.array(v, dtype=np.int32)


class Make:
    """The pricer over any backend with ``compile`` and ``run`` (the
    ``Make (B : Backend.S)`` functor, lsm.ml:245-315)."""

    def __init__(self, backend, n_paths, n_steps, m=market):
        if n_paths < 1 or n_steps < 1:
            raise ValueError("Lsm.create: n_paths and n_steps must be >= 1")
        self.b = backend
        self.n_paths, self.n_steps = n_paths, n_steps
        self.strike = m.strike
        self.disc = math.exp(-m.rate * (m.maturity / n_steps))
        self.paths = backend.compile(paths_graph(n_paths, n_steps, m))
        self.regress = backend.compile(regress_graph(n_paths, n_steps, self.strike, self.disc))
        self.update = backend.compile(update_graph(n_paths, n_steps, self.strike, self.disc))

    def price(self, seed):
        n, ns = self.n_paths, self.n_steps
        s = dict(self.b.run(self.paths, [("seed", _scalar_i32(seed))]))["S"]
        cf = np.maximum(self.strike - s[:, ns - 1], 0.0)
        for step in range(ns - 2, -1, -1):
            tv = _scalar_i32(step)
            outs = dict(self.b.run(self.regress, [("S", s), ("cf", cf), ("t", tv)]))
            beta = _beta(outs["xtx"], outs["xty"])
            cf = dict(self.b.run(self.update, [("S", s), ("cf", cf), ("t", tv), ("beta", beta)]))["cf"]
        return self.disc * (float(np.sum(cf)) / n)


class MakeResident:
    """The same algorithm on device-resident values (lsm.ml:318-409): S is
    produced and kept on the device, the cash flow never leaves it, and per
    step only xtx (9 doubles), xty (3), beta (3) and t cross the bus. The
    arithmetic is Make's, kernel for kernel, so the prices agree bit for
    bit."""

    def __init__(self, n_paths, n_steps, m=market):
        from .. import backend_hip as H

        if n_paths < 1 or n_steps < 1:
            raise ValueError("Lsm.Make_resident.create: n_paths and n_steps must be >= 1")
        self.H = H
        self.n_paths, self.n_steps = n_paths, n_steps
        self.strike = m.strike
        self.disc = math.exp(-m.rate * (m.maturity / n_steps))
        self.paths = H.compile(paths_graph(n_paths, n_steps, m))
        self.regress = H.compile(regress_graph(n_paths, n_steps, self.strike, self.disc))
        self.update = H.compile(update_graph(n_paths, n_steps, self.strike, self.disc))

    def price(self, seed):
        H = self.H
        ns = self.n_steps
        seed_r = H.upload(_scalar_i32(seed))
        s = dict(H.run_resident(self.paths, [("seed", seed_r)]))["S"]
        H.free_resident(seed_r)
        s_last = H.download(s)[:, ns - 1]
        cf = H.upload(np.maximum(self.strike - s_last, 0.0))
        for step in range(ns - 2, -1, -1):
            tv = H.upload(_scalar_i32(step))
            outs = dict(H.run_resident(self.regress, [("S", s), ("cf", cf), ("t", tv)]))
            xtx, xty = H.download(outs["xtx"]), H.download(outs["xty"])
            H.free_resident(outs["xtx"])
            H.free_resident(outs["xty"])
            bv = H.upload(_beta(xtx, xty))
            nxt = dict(H.run_resident(self.update, [("S", s), ("cf", cf), ("t", tv), ("beta", bv)]))["cf"]
            for r in (cf, tv, bv):
                H.free_resident(r)
            cf = nxt
        final = H.download(cf)
        H.free_resident(cf)
        H.free_resident(s)
        return self.disc * (float(np.sum(final)) / self.n_paths)

    def release(self):
        for c in (self.paths, self.regress, self.update):
            c.release()
