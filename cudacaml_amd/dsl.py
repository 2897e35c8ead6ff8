"""The user surface: tensor combinators and scalar expression builders.

Restates ``lib/ir/dsl.ml:1-196`` (the OCaml ``Dsl`` module) with the same
names, argument meaning, shape rules and ``Invalid_argument`` messages
(raised here as ``ValueError``). Python spellings that would shadow a
builtin keep the reference name anyway (``map``, ``min``, ``max``): import
the module qualified, ``from cudacaml_amd import dsl as D``.
"""

from __future__ import annotations

from . import ir
from .ir import BOOL, F32, F64, I32, I64, Expr, Tensor, numel, shape_to_string

# ---------------------------------------------------------------------------
# Tensors
# ---------------------------------------------------------------------------


def param(name, dtype, shape):
    return Tensor(dtype, shape, "param", pname=name)


def iota(shape):
    return Tensor(I32, shape, "iota")


def map(f, src):  # noqa: A001 - the reference name
    fn = ir.fn1(src.dtype, f)
    return Tensor(fn.body1.dtype, src.shape, "map", a=src, fn=fn)


def map2(f, a, b):
    # No broadcasting: both operands must have the same shape (dsl.ml:9-16).
    if a.shape != b.shape:
        raise ValueError(
            "Dsl.map2: shape mismatch: %s vs %s" % (shape_to_string(a.shape), shape_to_string(b.shape))
        )
    fn = ir.fn2(a.dtype, b.dtype, f)
    return Tensor(fn.body2.dtype, a.shape, "map2", a=a, b=b, fn=fn)


def gather(idx, src):
    return Tensor(src.dtype, idx.shape, "gather", a=idx, b=src)


def _accumulable(d):
    return d in (F32, F64, I32)


def scatter_add(idx, src, shape):
    if idx.shape != src.shape:
        raise ValueError(
            "Dsl.scatter_add: idx shape %s does not match src shape %s"
            % (shape_to_string(idx.shape), shape_to_string(src.shape))
        )
    if not _accumulable(src.dtype):
        raise ValueError("Dsl.scatter_add: dtype %s cannot be accumulated" % src.dtype.name)
    return Tensor(src.dtype, shape, "scatter_add", a=idx, b=src)


def reshape(shape, src):
    shape = tuple(shape)
    if numel(shape) != numel(src.shape):
        raise ValueError(
            "Dsl.reshape: numel mismatch: %s (%d) vs %s (%d)"
            % (shape_to_string(shape), numel(shape), shape_to_string(src.shape), numel(src.shape))
        )
    return Tensor(src.dtype, shape, "reshape", a=src)


def _all_but_last(dims):
    return tuple(dims[:-1]) if dims else ()


def flatten(src):
    return reshape((numel(src.shape),), src)


def reduce(f, init, src):
    """Whole-tensor reduction: flattens first, result shape [] (dsl.ml:65-73)."""
    fn = ir.fn2(src.dtype, src.dtype, f)
    if len(src.shape) == 1:
        return Tensor(src.dtype, (), "reduce", a=src, fn=fn, init=init)
    flat = flatten(src)
    return Tensor(src.dtype, (), "reduce", a=flat, fn=fn, init=init)


def scan(f, init, src):
    fn = ir.fn2(src.dtype, src.dtype, f)
    if len(src.shape) == 1:
        return Tensor(src.dtype, src.shape, "scan", a=src, fn=fn, init=init)
    flat = flatten(src)
    scanned = Tensor(src.dtype, flat.shape, "scan", a=flat, fn=fn, init=init)
    return reshape(src.shape, scanned)


def reduce_rows(f, init, src):
    if len(src.shape) < 2:
        raise ValueError("Dsl.reduce_rows: rank >= 2 required, got %s" % shape_to_string(src.shape))
    fn = ir.fn2(src.dtype, src.dtype, f)
    return Tensor(src.dtype, _all_but_last(src.shape), "reduce", a=src, fn=fn, init=init)


def scan_rows(f, init, src):
    if len(src.shape) < 2:
        raise ValueError("Dsl.scan_rows: rank >= 2 required, got %s" % shape_to_string(src.shape))
    fn = ir.fn2(src.dtype, src.dtype, f)
    return Tensor(src.dtype, src.shape, "scan", a=src, fn=fn, init=init)


def broadcast(shape, src):
    if numel(src.shape) != 1:
        raise ValueError(
            "Dsl.broadcast: source must have exactly one element: %s (%d)"
            % (shape_to_string(src.shape), numel(src.shape))
        )
    return Tensor(src.dtype, shape, "broadcast", a=src)


# ---------------------------------------------------------------------------
# Scalars
# ---------------------------------------------------------------------------


def const(dtype, v):
    return ir.make_const(dtype, v)


def index():
    return Expr(I32, "index")


def binop(op, a, b):
    return Expr(a.dtype, "bin", op=op, a=a, b=b)


def unop(op, a):
    return Expr(a.dtype, "un", op=op, a=a)


def cmp(op, a, b):
    return Expr(BOOL, "cmp", op=op, a=a, b=b)


def add(a, b):
    return binop("add", a, b)


def sub(a, b):
    return binop("sub", a, b)


def mul(a, b):
    return binop("mul", a, b)


def div(a, b):
    return binop("div", a, b)


def min(a, b):  # noqa: A001
    return binop("min", a, b)


def max(a, b):  # noqa: A001
    return binop("max", a, b)


def bit_and(a, b):
    return binop("and", a, b)


def bit_or(a, b):
    return binop("or", a, b)


def bit_xor(a, b):
    return binop("xor", a, b)


def shl(a, b):
    return binop("shl", a, b)


def shr(a, b):
    return binop("shr", a, b)


def neg(a):
    return unop("neg", a)


def sqrt(a):
    return unop("sqrt", a)


def exp(a):
    return unop("exp", a)


def log(a):
    return unop("log", a)


def abs(a):  # noqa: A001
    return unop("abs", a)


def sin(a):
    return unop("sin", a)


def cos(a):
    return unop("cos", a)


def erf(a):
    return unop("erf", a)


def erfinv(a):
    return unop("erfinv", a)


def lt(a, b):
    return cmp("lt", a, b)


def le(a, b):
    return cmp("le", a, b)


def eq(a, b):
    return cmp("eq", a, b)


def ne(a, b):
    return cmp("ne", a, b)


def gt(a, b):
    return cmp("gt", a, b)


def ge(a, b):
    return cmp("ge", a, b)


def and_(a, b):
    return Expr(BOOL, "logic", op="and", a=a, b=b)


def or_(a, b):
    return Expr(BOOL, "logic", op="or", a=a, b=b)


def not_(a):
    return Expr(BOOL, "not", a=a)


def select(c, a, b):
    return Expr(a.dtype, "select", a=c, b=a, c=b)


def cast(dtype, e):
    return Expr(dtype, "cast", a=e)


# ---------------------------------------------------------------------------
# Tensors built out of the above (dsl.ml:152-196)
# ---------------------------------------------------------------------------


def full(dtype, shape, v):
    return map(lambda _: const(dtype, v), iota(shape))


def scalar(name, dtype):
    return param(name, dtype, ir.SCALAR)


def transpose(x):
    """``out[k] = x[(k mod m) * n + k / m]`` for ``x : [m; n]``, spelled as
    a gather over a computed index, with mod written ``k - (k/m)*m``
    (dsl.ml:159-182)."""
    if len(x.shape) != 2:
        raise ValueError("Dsl.transpose: rank 2 required, got %s" % shape_to_string(x.shape))
    m, n = x.shape
    mi = const(I32, m)
    ni = const(I32, n)

    def f(k):
        q = div(k, mi)
        return add(mul(sub(k, mul(q, mi)), ni), q)

    idx = map(f, iota((n, m)))
    return gather(idx, x)


def matmul(a, b):
    if len(a.shape) == 2 and len(b.shape) == 2 and a.shape[1] == b.shape[0]:
        return Tensor(a.dtype, (a.shape[0], b.shape[1]), "matmul", a=a, b=b)
    raise ValueError(
        "Dsl.matmul: need [m; k] x [k; n], got %s x %s" % (shape_to_string(a.shape), shape_to_string(b.shape))
    )

