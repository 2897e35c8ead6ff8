"""Symbolic derivatives of scalar expressions, with the simplifier that
keeps them small.

Restates ``lib/ad/deriv.ml`` (``simplify`` at :88-150, ``deriv`` at
:156-214, ``subst``/``apply`` at :232-282). Only the behaviour the
gradient graphs depend on is kept; a derivative is a fresh expression
built through ``dsl`` so every node has a new uid.
"""

from __future__ import annotations

import math

from . import dsl as D
from .ir import BOOL, F32, F64, Expr

TWO_OVER_SQRT_PI = 2.0 / math.sqrt(math.pi)
SQRT_PI_OVER_TWO = math.sqrt(math.pi) / 2.0


def fconst(dt, v):
    if dt is F32 or dt is F64:
        return D.const(dt, v)
    raise ValueError("Deriv: dtype %s is not differentiable" % dt.name)


def _round_f32(x):
    import numpy as np

    return float(np.float32(x))


def _fold_arith(op, x, y):
    if op == "add":
        return x + y
    if op == "sub":
        return x - y
    if op == "mul":
        return x * y
    if op == "div":
        return None if y == 0.0 else x / y
    return None


def _is_lit(e, v):
    return e.kind == "const" and (e.dtype is F32 or e.dtype is F64) and e.value == v


def simplify(e):
    """Constant folding and the unit/zero rewrites of deriv.ml:88-150."""
    memo = {}

    def go(e):
        r = memo.get(e.uid)
        if r is not None:
            return r
        r = _simplify1(e, go)
        memo[e.uid] = r
        return r

    return go(e)


def _simplify1(e, go):
    dt = e.dtype
    k = e.kind
    if k in ("const", "arg", "index"):
        return e
    if k == "bin":
        a, b = go(e.a), go(e.b)
        if a.kind == "const" and b.kind == "const" and dt in (F32, F64):
            r = _fold_arith(e.op, a.value, b.value)
            if r is not None:
                return D.const(dt, _round_f32(r) if dt is F32 else r)
        op = e.op
        if op == "mul":
            if _is_lit(b, 0.0):
                return b
            if _is_lit(a, 0.0):
                return a
            if _is_lit(b, 1.0):
                return a
            if _is_lit(a, 1.0):
                return b
        elif op == "add":
            if _is_lit(b, 0.0):
                return a
            if _is_lit(a, 0.0):
                return b
        elif op == "sub":
            if _is_lit(b, 0.0):
                return a
            if _is_lit(a, 0.0):
                return Expr(dt, "un", op="neg", a=b)
        if a is e.a and b is e.b:
            return e
        return Expr(dt, "bin", op=op, a=a, b=b)
    if k == "un":
        a = go(e.a)
        if e.op == "neg" and a.kind == "un" and a.op == "neg":
            return a.a
        return e if a is e.a else Expr(dt, "un", op=e.op, a=a)
    if k in ("cmp", "logic"):
        a, b = go(e.a), go(e.b)
        return e if (a is e.a and b is e.b) else Expr(dt, k, op=e.op, a=a, b=b)
    if k == "not":
        a = go(e.a)
        return e if a is e.a else Expr(dt, "not", a=a)
    if k == "select":
        c, a, b = go(e.a), go(e.b), go(e.c)
        if a.uid == b.uid:
            return a
        if c is e.a and a is e.b and b is e.c:
            return e
        return Expr(dt, "select", a=c, b=a, c=b)
    if k == "cast":
        x = go(e.a)
        if x.dtype is dt:
            return x
        return e if x is e.a else Expr(dt, "cast", a=x)
    raise ValueError("Deriv.simplify: unknown kind %s" % k)


def _deriv(e, wrt, memo):
    r = memo.get(e.uid)
    if r is not None:
        return r
    r = _deriv1(e, wrt, memo)
    memo[e.uid] = r
    return r


def _deriv1(e, wrt, memo):
    dt = e.dtype
    k = e.kind

    def d(x):
        return _deriv(x, wrt, memo)

    if k == "const":
        return fconst(dt, 0.0)
    if k == "arg":
        return fconst(dt, 1.0 if e.arg == wrt else 0.0)
    if k == "index":
        return fconst(dt, 0.0)
    if k == "bin":
        a, b, op = e.a, e.b, e.op
        if op == "add":
            return D.add(d(a), d(b))
        if op == "sub":
            return D.sub(d(a), d(b))
        if op == "mul":
            return D.add(D.mul(d(a), b), D.mul(a, d(b)))
        if op == "div":
            return D.div(D.sub(D.mul(d(a), b), D.mul(a, d(b))), D.mul(b, b))
        if op == "min":
            return D.select(D.le(a, b), d(a), d(b))
        if op == "max":
            return D.select(D.ge(a, b), d(a), d(b))
        raise ValueError("Deriv.d: %s is integer only" % {"and": "bit_and", "or": "bit_or", "xor": "bit_xor"}.get(op, op))
    if k == "un":
        a, op = e.a, e.op
        da = d(a)
        if op == "neg":
            return D.neg(da)
        if op == "sqrt":
            return D.div(da, D.mul(fconst(dt, 2.0), D.sqrt(a)))
        if op == "exp":
            return D.mul(D.exp(a), da)
        if op == "log":
            return D.div(da, a)
        if op == "abs":
            return D.select(D.lt(a, fconst(dt, 0.0)), D.neg(da), da)
        if op == "sin":
            return D.mul(D.cos(a), da)
        if op == "cos":
            return D.mul(D.neg(D.sin(a)), da)
        if op == "erf":
            return D.mul(D.mul(fconst(dt, TWO_OVER_SQRT_PI), D.exp(D.neg(D.mul(a, a)))), da)
        if op == "erfinv":
            y = D.erfinv(a)
            return D.mul(D.mul(fconst(dt, SQRT_PI_OVER_TWO), D.exp(D.mul(y, y))), da)
    if k == "cmp":
        raise ValueError("Deriv.d: a comparison has dtype bool")
    if k == "logic":
        raise ValueError("Deriv.d: a logical operator has dtype bool")
    if k == "not":
        raise ValueError("Deriv.d: a negation has dtype bool")
    if k == "select":
        return D.select(e.a, d(e.b), d(e.c))
    if k == "cast":
        x = e.a
        if x.dtype.is_float:
            return D.cast(dt, d(x))
        return fconst(dt, 0.0)
    raise ValueError("Deriv.d: unknown kind %s" % k)


def d(e, wrt):
    """d e / d Arg(wrt), simplified (deriv.ml:216-221)."""
    if not e.dtype.is_float:
        raise ValueError("Deriv.d: expression has dtype %s, a float dtype is required" % e.dtype.name)
    return simplify(_deriv(e, wrt, {}))


def subst(args, e):
    """Replace ``Arg i`` by ``args[i]``; every node is rebuilt with a fresh
    uid (deriv.ml:232-259)."""
    memo = {}

    def go(x):
        r = memo.get(x.uid)
        if r is not None:
            return r
        k = x.kind
        dt = x.dtype
        if k == "arg":
            s = args.get(x.arg)
            if s is None:
                r = Expr(dt, "arg", arg=x.arg)
            else:
                if s.dtype is not dt:
                    raise ValueError(
                        "Deriv.apply: Arg %d has dtype %s but the substitute has dtype %s" % (x.arg, dt.name, s.dtype.name)
                    )
                r = s
        elif k == "const":
            r = Expr(dt, "const", value=x.value)
        elif k == "index":
            r = Expr(dt, "index")
        elif k in ("bin", "cmp", "logic"):
            r = Expr(dt, k, op=x.op, a=go(x.a), b=go(x.b))
        elif k == "un":
            r = Expr(dt, k, op=x.op, a=go(x.a))
        elif k in ("not", "cast"):
            r = Expr(dt, k, a=go(x.a))
        elif k == "select":
            r = Expr(dt, k, a=go(x.a), b=go(x.b), c=go(x.c))
        else:
            raise ValueError(k)
        memo[x.uid] = r
        return r

    return go(e)


def apply1(body, x):
    return subst({0: x}, body)


def apply2(body, x, y):
    return subst({0: x, 1: y}, body)


__all__ = ["d", "simplify", "subst", "apply1", "apply2", "fconst", "BOOL"]
