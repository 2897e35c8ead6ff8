"""Differential testing: run one graph on two backends and compare outputs.

``check`` restates ``lib/backend/differential.ml:6-88``: outputs are
compared by name (order is free, extra outputs are ignored, a missing one
is an error), dtype and shape must match, NaN equals NaN, floats must lie
in the band ``|g - e| <= tol * (1 + |e|)`` (default 1e-5), integers must be
equal, and a backend that raises yields an error rather than an exception.
The result is ``(True, None)`` or ``(False, message)``.

``policy_check`` adds the per-output bar of this backend: integer, Philox,
gather and cast results bit-exact; f32 element-wise results within 2 ulp;
results that pass through an f32 reduction, scan, matmul or scatter_add
within 1e-4 relative; f64 within 1e-12 relative.
"""

from __future__ import annotations

import numpy as np

from . import ir


def float_close(e, g, tolerance):
    e = np.asarray(e, dtype=np.float64)
    g = np.asarray(g, dtype=np.float64)
    both_nan = np.isnan(e) & np.isnan(g)
    with np.errstate(invalid="ignore"):
        ok = np.abs(g - e) <= tolerance * (1.0 + np.abs(e))
    return ok | both_nan


def _compare_one(name, e, g, tolerance):
    if e.dtype != g.dtype:
        return "output %s: dtype mismatch: expected %s, got %s" % (
            name, ir.dtype_of_numpy(e).name, (ir.dtype_of_numpy(g) or g.dtype).name if ir.dtype_of_numpy(g) else g.dtype)
    if e.shape != g.shape:
        return "output %s: shape mismatch: expected %s, got %s" % (
            name, ir.shape_to_string(e.shape), ir.shape_to_string(g.shape))
    ef = e.reshape(-1)
    gf = g.reshape(-1)
    if e.dtype.kind == "f":
        ok = float_close(ef, gf, tolerance)
    else:
        ok = ef == gf
    if not ok.all():
        i = int(np.argmin(ok))
        return "output %s[%d]: expected %g, got %g (tol %g)" % (name, i, float(ef[i]), float(gf[i]), tolerance)
    return None


def compare_all(expected, got, tolerance=1e-5):
    gd = {}
    for n, v in got:
        gd.setdefault(n, v)
    for n, e in expected:
        if n not in gd:
            return False, "missing output %s" % n
        msg = _compare_one(n, np.asarray(e), np.asarray(gd[n]), tolerance)
        if msg:
            return False, msg
    return True, None


def check(reference, candidate, graph, inputs, tolerance=1e-5):
    """``Differential.check ~reference ~candidate graph ~inputs``."""
    try:
        expected = reference.run(reference.compile(graph), inputs)
    except Exception as ex:  # noqa: BLE001 - a raising backend is a result
        return False, "%s raised: %s" % (reference.name, ex)
    try:
        got = candidate.run(candidate.compile(graph), inputs)
    except Exception as ex:  # noqa: BLE001
        return False, "%s raised: %s" % (candidate.name, ex)
    return compare_all(expected, got, tolerance)


# ---------------------------------------------------------------------------
# The per-output bar
# ---------------------------------------------------------------------------

ULP_F32 = 2
TOL_F32_ACCUM = 1e-4
TOL_F64 = 1e-12


def accumulates(t):
    """True if a float output passes through an order-dependent f32/f64
    accumulation: Reduce, Scan, Matmul or a float Scatter_add."""
    seen = set()
    stack = [t]
    while stack:
        n = stack.pop()
        if n.uid in seen:
            continue
        seen.add(n.uid)
        if n.kind in ("reduce", "scan", "matmul") and n.dtype.is_float:
            return True
        if n.kind == "scatter_add" and n.dtype.is_float:
            return True
        stack.extend(n.deps())
    return False


def ulp_distance_f32(e, g):
    """|ordinal(e) - ordinal(g)| for float32 bit patterns (NaN==NaN -> 0)."""
    ei = np.asarray(e, dtype=np.float32).view(np.int32).astype(np.int64)
    gi = np.asarray(g, dtype=np.float32).view(np.int32).astype(np.int64)
    eo = np.where(ei < 0, -(ei & 0x7FFFFFFF), ei)
    go = np.where(gi < 0, -(gi & 0x7FFFFFFF), gi)
    d = np.abs(eo - go)
    both_nan = np.isnan(np.asarray(e, dtype=np.float32)) & np.isnan(np.asarray(g, dtype=np.float32))
    return np.where(both_nan, 0, d)


class Verdict:
    __slots__ = ("name", "rule", "ok", "failures", "worst", "message")

    def __init__(self, name, rule, ok, failures, worst, message):
        self.name = name
        self.rule = rule
        self.ok = ok
        self.failures = failures
        self.worst = worst
        self.message = message

    def __repr__(self):
        return "Verdict(%s %s ok=%s failures=%d worst=%g%s)" % (
            self.name, self.rule, self.ok, self.failures, self.worst, "" if not self.message else " " + self.message)


def rule_for(t):
    if not t.dtype.is_float:
        return "exact"
    if t.dtype is ir.F64:
        return "rel1e-12"
    return "rel1e-4" if accumulates(t) else "ulp2"


def verdict(name, rule, e, g):
    e = np.asarray(e)
    g = np.asarray(g)
    if e.dtype != g.dtype or e.shape != g.shape:
        return Verdict(name, rule, False, -1, float("inf"), "dtype/shape mismatch %s%s vs %s%s" % (
            e.dtype, e.shape, g.dtype, g.shape))
    ef = e.reshape(-1)
    gf = g.reshape(-1)
    if ef.size == 0:
        return Verdict(name, rule, True, 0, 0.0, None)
    if rule == "exact":
        bad = ef != gf
        worst = float(np.max(np.abs(ef.astype(np.float64) - gf.astype(np.float64)))) if bad.any() else 0.0
    elif rule == "ulp2":
        d = ulp_distance_f32(ef, gf)
        bad = d > ULP_F32
        worst = float(d.max())
    else:
        tol = TOL_F64 if rule == "rel1e-12" else TOL_F32_ACCUM
        e64 = ef.astype(np.float64)
        g64 = gf.astype(np.float64)
        with np.errstate(invalid="ignore"):
            ratio = np.abs(g64 - e64) / (tol * (1.0 + np.abs(e64)))
        # equal values (infinities included) and NaN against NaN agree
        ratio = np.where((e64 == g64) | (np.isnan(e64) & np.isnan(g64)), 0.0, ratio)
        ratio = np.where(np.isnan(ratio), np.inf, ratio)
        bad = ratio > 1.0
        worst = float(ratio.max())
    n_bad = int(bad.sum())
    msg = None
    if n_bad:
        i = int(np.argmax(bad))
        msg = "first failure at %d: expected %r, got %r" % (i, ef[i].item(), gf[i].item())
    return Verdict(name, rule, n_bad == 0, n_bad, worst, msg)


def policy_check(graph, expected, got):
    """One ``Verdict`` per graph output, by name."""
    gd = dict(got)
    out = []
    for n, t in graph.outputs:
        e = dict(expected)[n]
        if n not in gd:
            out.append(Verdict(n, rule_for(t), False, -1, float("inf"), "missing output"))
            continue
        out.append(verdict(n, rule_for(t), e, gd[n]))
    return out
