"""Black-Scholes: a European call priced by Monte Carlo, with pathwise
Greeks from ``grad`` (examples/black_scholes.ml:31-166).

Three graphs: ``call_mc`` (one-step GBM), ``call_mc_paths`` (an n-step path
built with ``scan_rows`` over log-increments, then the last column by a
gather) and ``call_greeks`` (call_mc plus d/ds0, d/dvol, d/drate).
"""

from __future__ import annotations

import math

import numpy as np

from .. import dsl as D
from .. import grad as G
from .. import rng
from ..ir import F64, I32, Graph


class Market:
    __slots__ = ("s0", "strike", "vol", "rate", "maturity")

    def __init__(self, s0=100.0, strike=100.0, vol=0.2, rate=0.05, maturity=1.0):
        self.s0 = s0
        self.strike = strike
        self.vol = vol
        self.rate = rate
        self.maturity = maturity


market = Market()


def norm_cdf(x):
    return 0.5 * (1.0 + math.erf(x / math.sqrt(2.0)))


def norm_pdf(x):
    return math.exp(-0.5 * x * x) / math.sqrt(2.0 * math.pi)


def analytic(m=market):
    """The textbook call price with delta, vega and rho (black_scholes.ml:44-58)."""
    sqrt_t = math.sqrt(m.maturity)
    d1 = (math.log(m.s0 / m.strike) + (m.rate + 0.5 * m.vol * m.vol) * m.maturity) / (m.vol * sqrt_t)
    d2 = d1 - m.vol * sqrt_t
    disc = math.exp(-m.rate * m.maturity)
    return {
        "price": m.s0 * norm_cdf(d1) - m.strike * disc * norm_cdf(d2),
        "delta": norm_cdf(d1),
        "vega": m.s0 * norm_pdf(d1) * sqrt_t,
        "rho": m.strike * m.maturity * disc * norm_cdf(d2),
    }


def _params(dtype):
    return D.scalar("s0", dtype), D.scalar("vol", dtype), D.scalar("rate", dtype), D.scalar("seed", I32)


def discounted_mean(dtype, n_paths, m, st, rate):
    kf = lambda v: D.const(dtype, v)  # noqa: E731
    payoff = D.map(lambda s: D.max(D.sub(s, kf(m.strike)), kf(0.0)), st)
    total = D.reduce(D.add, kf(0.0), payoff)
    mean = D.map(lambda s: D.div(s, kf(float(n_paths))), total)
    return D.map2(lambda mu, r: D.mul(mu, D.exp(D.neg(D.mul(r, kf(m.maturity))))), mean, rate)


def call_mc(n_paths, dtype, m=market):
    shape = (n_paths,)
    s0, vol, rate, seed = _params(dtype)
    kf = lambda v: D.const(dtype, v)  # noqa: E731
    z = rng.normal(dtype, seed, shape)
    s0b = D.broadcast(shape, s0)
    volb = D.broadcast(shape, vol)
    rateb = D.broadcast(shape, rate)
    drift = D.map2(lambda r, v: D.mul(D.sub(r, D.mul(kf(0.5), D.mul(v, v))), kf(m.maturity)), rateb, volb)
    diffusion = D.map2(lambda v, zi: D.mul(D.mul(v, kf(math.sqrt(m.maturity))), zi), volb, z)
    st = D.map2(lambda s, e: D.mul(s, D.exp(e)), s0b, D.map2(D.add, drift, diffusion))
    return Graph.create("bs_mc", [("price", discounted_mean(dtype, n_paths, m, st, rate))])


def call_mc_paths(n_paths, n_steps, dtype, m=market, draws=None):
    """``draws`` (a test hook, not in the reference): a tensor of the grid's
    shape used in place of the Philox normal draws, e.g. a param."""
    grid = (n_paths, n_steps)
    s0, vol, rate, seed = _params(dtype)
    kf = lambda v: D.const(dtype, v)  # noqa: E731
    ki = lambda v: D.const(I32, v)  # noqa: E731
    dt = m.maturity / float(n_steps)
    z = rng.normal(dtype, seed, grid) if draws is None else draws
    s0b = D.broadcast(grid, s0)
    volb = D.broadcast(grid, vol)
    rateb = D.broadcast(grid, rate)
    drift = D.map2(lambda r, v: D.mul(D.sub(r, D.mul(kf(0.5), D.mul(v, v))), kf(dt)), rateb, volb)
    diffusion = D.map2(lambda v, zi: D.mul(D.mul(v, kf(math.sqrt(dt))), zi), volb, z)
    cum = D.scan_rows(D.add, kf(0.0), D.map2(D.add, drift, diffusion))
    paths = D.map(D.exp, D.map2(lambda s, c: D.add(D.log(s), c), s0b, cum))
    idx = D.map(lambda p: D.add(D.mul(p, ki(n_steps)), ki(n_steps - 1)), D.iota((n_paths,)))
    st = D.gather(idx, paths)
    return Graph.create("bs_paths", [("price", discounted_mean(dtype, n_paths, m, st, rate))])


def call_greeks(n_paths, dtype, m=market):
    return G.grad(call_mc(n_paths, dtype, m), "price", ["s0", "vol", "rate"])


def call_paths_greeks(n_paths, n_steps, dtype, m=market, wrt=("s0", "vol"), draws=None):
    """The multi-step pricer differentiated: delta and vega (and rho if asked)."""
    return G.grad(call_mc_paths(n_paths, n_steps, dtype, m, draws), "price", list(wrt))


def inputs(dtype, m=market, seed=7):
    return [
        ("s0", np.array(m.s0, dtype=dtype.np)),
        ("vol", np.array(m.vol, dtype=dtype.np)),
        ("rate", np.array(m.rate, dtype=dtype.np)),
        ("seed", np.array(seed, dtype=np.int32)),
    ]


def scalar_out(outs, name):
    for n, v in outs:
        if n == name:
            if v.dtype.kind != "f":
                raise ValueError("Black_scholes.scalar_out: output %r is not a float" % name)
            return float(v.reshape(-1)[0])
    raise KeyError(name)


__all__ = ["Market", "market", "analytic", "call_mc", "call_mc_paths", "call_greeks", "inputs", "scalar_out", "F64"]
