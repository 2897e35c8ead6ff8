"""Reverse-mode differentiation of a graph, as a graph-to-graph transform.

Restates ``lib/ad/grad.ml``: one reverse walk of the topological order with
a table of adjoints keyed by uid (``grad.ml:334-348``), one rule per node
kind (``grad.ml:211-305``). Everything built here comes from ``dsl``, so
the gradient graph contains only node kinds the backend already runs:
Reduce-add spreads by a gather, Scan-add becomes total - prefix + abar,
Gather becomes Scatter_add, Matmul becomes two Matmuls over transposes.
"""

from __future__ import annotations

from . import deriv as Deriv
from . import dsl as D
from .ir import F32, F64, I32, I64, Graph, row_length


class NotDifferentiable(Exception):
    pass


def grad_name(output, wrt):
    return "d" + output + "/d" + wrt


def _fconst(dt, v):
    if dt is F32 or dt is F64:
        return D.const(dt, v)
    raise NotDifferentiable("dtype %s carries no gradient" % dt.name)


def _fones(dt, shape):
    if dt is F32 or dt is F64:
        return D.full(dt, shape, 1.0)
    raise NotDifferentiable("dtype %s carries no gradient" % dt.name)


def _zeros(dt, shape):
    if dt in (F32, F64, I32, I64):
        return D.full(dt, shape, 0)
    raise ValueError("Grad.grad: a bool tensor cannot hold a gradient")


class _Tbl:
    def __init__(self):
        self.adj = {}

    def find(self, node):
        a = self.adj.get(node.uid)
        if a is not None and a.dtype is not node.dtype:
            raise ValueError("Grad: internal adjoint dtype mismatch")
        return a

    def accumulate(self, node, v):
        a = self.find(node)
        self.adj[node.uid] = v if a is None else D.map2(D.add, a, v)

    def accum_into(self, tgt, v):
        if tgt.dtype.is_float:
            if tgt.dtype is v.dtype:
                self.accumulate(tgt, v)
            else:
                self.accumulate(tgt, D.map(lambda e: D.cast(tgt.dtype, e), v))


def _dbody1(what, body):
    try:
        return Deriv.d(body, 0)
    except ValueError as m:
        raise NotDifferentiable(what + ": " + str(m))


def _dbody2(what, body, wrt):
    try:
        return Deriv.d(body, wrt)
    except ValueError as m:
        raise NotDifferentiable(what + ": " + str(m))


_BINOP_NAME = {
    "add": "Add", "sub": "Sub", "mul": "Mul", "div": "Div", "min": "Min", "max": "Max",
    "and": "Bit_and", "or": "Bit_or", "xor": "Bit_xor", "shl": "Shl", "shr": "Shr",
}


def _is_arg(e, i):
    return e.kind == "arg" and e.arg == i


def combining_binop(fn):
    """The one binop over the two placeholders, in either order, or None
    (grad.ml:154-166)."""
    b = fn.body2
    if b.kind == "bin":
        if (_is_arg(b.a, 0) and _is_arg(b.b, 1)) or (_is_arg(b.a, 1) and _is_arg(b.b, 0)):
            return b.op
    return None


def _op_desc(kind, op):
    if op is None:
        return "%s <unrecognised operator>" % kind
    return "%s %s" % (kind, _BINOP_NAME[op])


def _rows_of(src_shape, t):
    """``out[k] = t[k / n]``: a row-shaped tensor replicated over the source
    (grad.ml:179-189)."""
    n = row_length(src_shape)
    ni = D.const(I32, n)
    idx = D.map(lambda k: D.div(k, ni), D.iota(src_shape))
    return D.gather(idx, t)


def _reduce_last(t):
    init = _fconst(t.dtype, 0.0)
    if len(t.shape) <= 1:
        return D.reduce(D.add, init, t)
    return D.reduce_rows(D.add, init, t)


def _scan_last(t):
    init = _fconst(t.dtype, 0.0)
    if len(t.shape) <= 1:
        return D.scan(D.add, init, t)
    return D.scan_rows(D.add, init, t)


def _back_node(tbl, t, abar):
    k = t.kind
    if k in ("param", "iota"):
        return
    if k == "map":
        src = t.a
        if src.dtype.is_float:
            df = _dbody1("Map", t.fn.body1)
            tbl.accum_into(src, D.map2(lambda adj, x: D.mul(adj, Deriv.apply1(df, x)), abar, src))
        return
    if k == "map2":
        xa, xb = t.a, t.b
        for wrt, tgt in ((0, xa), (1, xb)):
            if tgt.dtype.is_float:
                df = _dbody2("Map2", t.fn.body2, wrt)
                dk = D.map2(lambda x, y, df=df: Deriv.apply2(df, x, y), xa, xb)
                tbl.accum_into(tgt, D.map2(D.mul, abar, dk))
        return
    if k == "reduce":
        src = t.a

        def spread(u):
            return _rows_of(src.shape, u)

        op = combining_binop(t.fn)
        if op == "add":
            tbl.accum_into(src, spread(abar))
        elif op in ("max", "min"):
            # Every element equal to the extremum receives the whole adjoint.
            m = spread(t)
            one = _fconst(t.dtype, 1.0)
            zero = _fconst(t.dtype, 0.0)
            mask = D.map2(lambda x, mv: D.select(D.eq(x, mv), one, zero), src, m)
            tbl.accum_into(src, D.map2(D.mul, spread(abar), mask))
        elif op == "mul":
            q = D.map2(D.div, spread(t), src)
            tbl.accum_into(src, D.map2(D.mul, spread(abar), q))
        else:
            raise NotDifferentiable(_op_desc("Reduce", op))
        return
    if k == "scan":
        src = t.a
        op = combining_binop(t.fn)
        if op == "add":
            total = _rows_of(src.shape, _reduce_last(abar))
            prefix = _scan_last(abar)
            tbl.accum_into(src, D.map2(D.add, D.map2(D.sub, total, prefix), abar))
        else:
            raise NotDifferentiable(_op_desc("Scan", op))
        return
    if k == "gather":
        idx, src = t.a, t.b
        if src.dtype.is_float:
            tbl.accumulate(src, D.scatter_add(idx, abar, src.shape))
        return
    if k == "scatter_add":
        idx, src = t.a, t.b
        tbl.accum_into(src, D.gather(idx, abar))
        return
    if k == "matmul":
        xa, xb = t.a, t.b
        if xa.dtype.is_float:
            tbl.accum_into(xa, D.matmul(abar, D.transpose(xb)))
        if xb.dtype.is_float:
            tbl.accum_into(xb, D.matmul(D.transpose(xa), abar))
        return
    if k == "reshape":
        src = t.a
        tbl.accum_into(src, D.reshape(src.shape, abar))
        return
    if k == "broadcast":
        src = t.a
        total = D.reduce(D.add, _fconst(t.dtype, 0.0), abar)
        tbl.accum_into(src, D.reshape(src.shape, total))
        return
    raise ValueError("Grad: unknown node kind %s" % k)


def grad(g, output, wrt):
    """The graph's outputs followed by ``d<output>/d<p>`` for each ``p`` in
    ``wrt`` (grad.ml:334-348)."""
    outs = list(g.outputs)
    params = dict(g.params)
    out = None
    for n, t in outs:
        if n == output:
            out = t
            break
    if out is None:
        raise ValueError("Grad.grad: no output named %r" % output)
    wrt_nodes = []
    for p in wrt:
        if p not in params:
            raise ValueError("Grad.grad: no param named %r" % p)
        wrt_nodes.append((p, params[p]))
    tbl = _Tbl()
    if not out.dtype.is_float:
        raise ValueError("Grad.grad: output has dtype %s, a float dtype is required" % out.dtype.name)
    tbl.accumulate(out, _fones(out.dtype, out.shape))
    for t in reversed(g.order):
        abar = tbl.find(t)
        if abar is not None:
            _back_node(tbl, t, abar)
    grads = []
    for p, node in wrt_nodes:
        a = tbl.find(node)
        grads.append((grad_name(output, p), a if a is not None else _zeros(node.dtype, node.shape)))
    return Graph.create(g.name + "_grad", outs + grads)
