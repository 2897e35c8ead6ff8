"""The array IR the backend serves: dtypes, shapes, scalar expressions,
tensor nodes and whole graphs, plus the text wire format both the HIP
backend and the CPU oracle read.

This is a host-side restatement of the reference front end, which stays in
OCaml upstream: ``lib/ir/dtype.ml:9-46``, ``lib/ir/shape.ml``,
``lib/ir/expr.ml:13-64``, ``lib/ir/tensor.ml:13-65`` and
``lib/ir/graph.ml:53-103``. Node identity is a process-wide ``uid``, as in
``lib/ir/uid.ml``; every table below is keyed by it and never by structure.

The wire format (one graph per text, version 1) is what an OCaml
``Backend_hip`` would print from a ``Graph.t`` before handing it to the
C-ABI; ``to_wire`` is the Python side of that contract::

    cchip-graph 1 <name>
    x <eid> <kind> <dtype> <fields...>          scalar expression node
    t <tid> <kind> <dtype> <rank> <dims...> <fields...>   tensor node
    o <name> <tid>                              graph output, in order
    end

Expression nodes precede their first use and are shared (a DAG), tensor
nodes are in the graph's topological order. Float constants are written as
the 16 hex digits of the IEEE double, because an F32 ``Const`` carries the
OCaml double unrounded (``cudacaml_backend_interp.ml:246``).
"""

from __future__ import annotations

import itertools
import struct

import numpy as np

# ---------------------------------------------------------------------------
# Dtypes  (lib/ir/dtype.ml:9-46)
# ---------------------------------------------------------------------------


class Dtype:
    __slots__ = ("name", "size", "is_float", "np", "code")

    def __init__(self, name, size, is_float, npdt, code):
        self.name = name
        self.size = size
        self.is_float = is_float
        self.np = npdt
        self.code = code

    def __repr__(self):
        return "Dtype." + self.name.upper()


F32 = Dtype("f32", 4, True, np.dtype(np.float32), 0)
F64 = Dtype("f64", 8, True, np.dtype(np.float64), 1)
I32 = Dtype("i32", 4, False, np.dtype(np.int32), 2)
I64 = Dtype("i64", 8, False, np.dtype(np.int64), 3)
BOOL = Dtype("bool", 1, False, np.dtype(np.bool_), 4)

DTYPES = (F32, F64, I32, I64, BOOL)
_BY_NAME = {d.name: d for d in DTYPES}
_BY_CODE = {d.code: d for d in DTYPES}


def dtype_of_name(name):
    return _BY_NAME[name]


def dtype_of_code(code):
    return _BY_CODE[code]


def dtype_of_numpy(a):
    """The storable dtype of a numpy array, or ``None``."""
    for d in (F32, F64, I32, I64):
        if a.dtype == d.np:
            return d
    return None


# ---------------------------------------------------------------------------
# Shapes  (lib/ir/shape.ml)
# ---------------------------------------------------------------------------

SCALAR = ()


def numel(shape):
    n = 1
    for d in shape:
        n *= d
    return n


def shape_to_string(shape):
    return "[" + ",".join(str(d) for d in shape) + "]"


def row_length(shape):
    """Extent of the last axis; a rank-0 shape is one row of one element
    (``cudacaml_backend_interp.ml:269-270``)."""
    return shape[-1] if len(shape) else 1


# ---------------------------------------------------------------------------
# Uids  (lib/ir/uid.ml)
# ---------------------------------------------------------------------------

_counter = itertools.count(1)


def fresh_uid():
    return next(_counter)


# ---------------------------------------------------------------------------
# Scalar expressions  (lib/ir/expr.ml:13-64)
# ---------------------------------------------------------------------------

BINOPS = ("add", "sub", "mul", "div", "min", "max", "and", "or", "xor", "shl", "shr")
INT_ONLY_BINOPS = ("and", "or", "xor", "shl", "shr")
UNOPS = ("neg", "sqrt", "exp", "log", "abs", "sin", "cos", "erf", "erfinv")
FLOAT_ONLY_UNOPS = ("sqrt", "exp", "log", "sin", "cos", "erf", "erfinv")
CMPS = ("eq", "ne", "lt", "le", "gt", "ge")
LOGICS = ("and", "or")


def wrap_i32(v):
    v = int(v) & 0xFFFFFFFF
    return v - (1 << 32) if v >= (1 << 31) else v


def wrap_i64(v):
    v = int(v) & 0xFFFFFFFFFFFFFFFF
    return v - (1 << 64) if v >= (1 << 63) else v


class Expr:
    """One scalar expression node. ``kind`` is one of const, arg, index,
    bin, un, cmp, logic, not, select, cast. Operands live in ``a``, ``b``,
    ``c``; ``op`` names the operator; ``value`` holds a constant and
    ``arg`` the placeholder position."""

    __slots__ = ("uid", "dtype", "kind", "op", "a", "b", "c", "value", "arg")

    def __init__(self, dtype, kind, op=None, a=None, b=None, c=None, value=None, arg=None):
        self.uid = fresh_uid()
        self.dtype = dtype
        self.kind = kind
        self.op = op
        self.a = a
        self.b = b
        self.c = c
        self.value = value
        self.arg = arg

    def operands(self):
        return [x for x in (self.a, self.b, self.c) if x is not None]

    def __repr__(self):
        return "Expr(%s %s %s)" % (self.kind, self.op or "", self.dtype.name)


def make_const(dtype, v):
    if dtype is F32 or dtype is F64:
        v = float(v)
    elif dtype is I32:
        v = wrap_i32(v)
    elif dtype is I64:
        v = wrap_i64(v)
    elif dtype is BOOL:
        v = bool(v)
    return Expr(dtype, "const", value=v)


class Fn1:
    """``('a, 'b) Expr.fn1``: the placeholder and the body built from it
    (``expr.ml:52-56``)."""

    __slots__ = ("arg1", "body1")

    def __init__(self, arg1, body1):
        self.arg1 = arg1
        self.body1 = body1


class Fn2:
    __slots__ = ("arg_a", "arg_b", "body2")

    def __init__(self, arg_a, arg_b, body2):
        self.arg_a = arg_a
        self.arg_b = arg_b
        self.body2 = body2


def fn1(dtype, f):
    a = Expr(dtype, "arg", arg=0)
    return Fn1(a, f(a))


def fn2(da, db, f):
    a = Expr(da, "arg", arg=0)
    b = Expr(db, "arg", arg=1)
    return Fn2(a, b, f(a, b))


# ---------------------------------------------------------------------------
# Tensors  (lib/ir/tensor.ml:13-65)
# ---------------------------------------------------------------------------

TENSOR_KINDS = (
    "param", "iota", "map", "map2", "reduce", "scan", "gather",
    "scatter_add", "matmul", "reshape", "broadcast",
)


class Tensor:
    """One tensor node. ``a``/``b`` are tensor operands in argument order,
    ``fn`` the element function (Fn1 for map, Fn2 for map2/reduce/scan),
    ``init`` the reduce/scan identity and ``pname`` a param's name."""

    __slots__ = ("uid", "dtype", "shape", "kind", "a", "b", "fn", "init", "pname")

    def __init__(self, dtype, shape, kind, a=None, b=None, fn=None, init=None, pname=None):
        self.uid = fresh_uid()
        self.dtype = dtype
        self.shape = tuple(int(d) for d in shape)
        self.kind = kind
        self.a = a
        self.b = b
        self.fn = fn
        self.init = init
        self.pname = pname

    def deps(self):
        """Direct data dependencies in argument order (``tensor.ml:49-65``)."""
        k = self.kind
        if k in ("param", "iota"):
            return []
        if k in ("map", "reduce", "scan", "reshape", "broadcast"):
            return [self.a]
        return [self.a, self.b]

    @property
    def numel(self):
        return numel(self.shape)

    def __repr__(self):
        return "Tensor(n%d %s %s %s)" % (self.uid, self.kind, shape_to_string(self.shape), self.dtype.name)


# ---------------------------------------------------------------------------
# Graphs  (lib/ir/graph.ml:53-103)
# ---------------------------------------------------------------------------


def _topo_sort(outputs):
    """Depth-first post-order from the outputs in list order, deps in
    argument order (``graph.ml:249-261``). Iterative, so a chain of a few
    thousand maps does not hit Python's recursion limit."""
    visited = set()
    order = []
    for _, root in outputs:
        if root.uid in visited:
            continue
        visited.add(root.uid)
        stack = [(root, iter(root.deps()))]
        while stack:
            node, it = stack[-1]
            nxt = None
            for d in it:
                if d.uid not in visited:
                    nxt = d
                    break
            if nxt is None:
                stack.pop()
                order.append(node)
            else:
                visited.add(nxt.uid)
                stack.append((nxt, iter(nxt.deps())))
    return order


class Graph:
    __slots__ = ("name", "outputs", "params", "order", "fan_out")

    def __init__(self, name, outputs, params, order, fan_out):
        self.name = name
        self.outputs = outputs
        self.params = params
        self.order = order
        self.fan_out = fan_out

    @staticmethod
    def create(name, outputs):
        outputs = [(str(n), t) for n, t in outputs]
        if not outputs:
            raise ValueError("Graph.create: a graph needs at least one output")
        seen = set()
        for n, _ in outputs:
            if n in seen:
                raise ValueError("Graph.create: duplicate output name %r" % n)
            seen.add(n)
        order = _topo_sort(outputs)
        params = []
        names = {}
        for t in order:
            if t.kind == "param":
                u = names.get(t.pname)
                if u is not None and u != t.uid:
                    raise ValueError("Graph.create: two Param nodes named %s" % t.pname)
                names[t.pname] = t.uid
                params.append((t.pname, t))
        # Counts USES (edges), not distinct consumers (graph.ml:263-276).
        fan = {}
        for t in order:
            for d in t.deps():
                fan[d.uid] = fan.get(d.uid, 0) + 1
        return Graph(name, outputs, params, order, fan)

    def fan_out_of(self, t):
        return self.fan_out.get(t.uid, 0)

    def param(self, name):
        for n, t in self.params:
            if n == name:
                return t
        raise KeyError(name)

    def output(self, name):
        for n, t in self.outputs:
            if n == name:
                return t
        raise KeyError(name)

    def to_dot(self):
        lines = ['digraph "%s" {' % self.name.replace('"', '\\"')]
        for t in self.order:
            kind = "Param " + t.pname if t.kind == "param" else _KIND_TITLE[t.kind]
            lines.append('  n%d [label="n%d %s %s %s"];' % (t.uid, t.uid, kind, shape_to_string(t.shape), t.dtype.name))
        for t in self.order:
            for d in t.deps():
                lines.append("  n%d -> n%d;" % (d.uid, t.uid))
        lines.append("}")
        return "\n".join(lines) + "\n"

    def to_wire(self):
        return to_wire(self)


_KIND_TITLE = {
    "param": "Param", "iota": "Iota", "map": "Map", "map2": "Map2", "reduce": "Reduce",
    "scan": "Scan", "gather": "Gather", "scatter_add": "Scatter_add", "matmul": "Matmul",
    "reshape": "Reshape", "broadcast": "Broadcast",
}


# ---------------------------------------------------------------------------
# Wire format
# ---------------------------------------------------------------------------


def escape_name(s):
    """Names travel as one whitespace-free token: '%', controls, spaces and
    non-ASCII bytes are percent-encoded; the empty name is a lone '%'."""
    if s == "":
        return "%"
    out = []
    for byte in s.encode("utf-8"):
        ch = chr(byte)
        if ch == "%" or byte <= 32 or byte >= 127:
            out.append("%%%02X" % byte)
        else:
            out.append(ch)
    return "".join(out)


def _const_token(e):
    d = e.dtype
    if d is F32 or d is F64:
        return "%016x" % struct.unpack("<Q", struct.pack("<d", e.value))[0]
    if d is BOOL:
        return "1" if e.value else "0"
    return str(int(e.value))


def _expr_lines(root, seen, lines):
    """Post-order, shared nodes once."""
    if root.uid in seen:
        return
    stack = [(root, False)]
    while stack:
        e, done = stack.pop()
        if e.uid in seen:
            continue
        if not done:
            stack.append((e, True))
            for o in reversed(e.operands()):
                if o.uid not in seen:
                    stack.append((o, False))
            continue
        seen.add(e.uid)
        k = e.kind
        head = "x %d %s %s" % (e.uid, k, e.dtype.name)
        if k == "const":
            lines.append(head + " " + _const_token(e))
        elif k == "arg":
            lines.append(head + " %d" % e.arg)
        elif k == "index":
            lines.append(head)
        elif k in ("bin", "cmp", "logic"):
            lines.append(head + " %s %d %d" % (e.op, e.a.uid, e.b.uid))
        elif k == "un":
            lines.append(head + " %s %d" % (e.op, e.a.uid))
        elif k in ("not", "cast"):
            lines.append(head + " %d" % e.a.uid)
        elif k == "select":
            lines.append(head + " %d %d %d" % (e.a.uid, e.b.uid, e.c.uid))
        else:
            raise ValueError("to_wire: unknown expression kind %s" % k)


def to_wire(g):
    lines = ["cchip-graph 1 " + escape_name(g.name)]
    seen = set()
    for t in g.order:
        if t.kind == "map":
            _expr_lines(t.fn.body1, seen, lines)
        elif t.kind == "map2":
            _expr_lines(t.fn.body2, seen, lines)
        elif t.kind in ("reduce", "scan"):
            _expr_lines(t.init, seen, lines)
            _expr_lines(t.fn.body2, seen, lines)
        head = "t %d %s %s %d%s" % (
            t.uid, t.kind, t.dtype.name, len(t.shape),
            "".join(" %d" % d for d in t.shape),
        )
        k = t.kind
        if k == "param":
            lines.append(head + " " + escape_name(t.pname))
        elif k == "iota":
            lines.append(head)
        elif k == "map":
            lines.append(head + " %d %d" % (t.a.uid, t.fn.body1.uid))
        elif k == "map2":
            lines.append(head + " %d %d %d" % (t.a.uid, t.b.uid, t.fn.body2.uid))
        elif k in ("reduce", "scan"):
            lines.append(head + " %d %d %d" % (t.a.uid, t.init.uid, t.fn.body2.uid))
        elif k in ("gather", "scatter_add", "matmul"):
            lines.append(head + " %d %d" % (t.a.uid, t.b.uid))
        elif k in ("reshape", "broadcast"):
            lines.append(head + " %d" % t.a.uid)
        else:
            raise ValueError("to_wire: unknown tensor kind %s" % k)
    for n, t in g.outputs:
        lines.append("o %s %d" % (escape_name(n), t.uid))
    lines.append("end")
    return "\n".join(lines) + "\n"
