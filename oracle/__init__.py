"""The CPU oracle, seen from Python: ``Interp``, a ``Backend.S``-shaped
wrapper over ``oracle/interp.c`` (the C restatement of
``lib/backend_interp/cudacaml_backend_interp.ml``).

TEST INFRASTRUCTURE ONLY. ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, as the checker and
nothing else; the product (``cudacaml_amd``) never does.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from cudacaml_amd import ir

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def build():
    """Compile ``oracle/interp.c`` with the committed Makefile."""
    subprocess.run(["make", "-B", "-s", "-C", _HERE], check=True)


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    lib.orc_parse.restype = ctypes.c_void_p
    lib.orc_parse.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int]
    lib.orc_free.argtypes = [ctypes.c_void_p]
    lib.orc_run.restype = ctypes.c_void_p
    lib.orc_run.argtypes = [
        ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_int),
        ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.POINTER(ctypes.c_int64)),
        ctypes.POINTER(ctypes.c_void_p), ctypes.c_char_p, ctypes.c_int,
    ]
    lib.orc_result_free.argtypes = [ctypes.c_void_p]
    lib.orc_result_count.argtypes = [ctypes.c_void_p]
    lib.orc_result_name.restype = ctypes.c_char_p
    lib.orc_result_name.argtypes = [ctypes.c_void_p, ctypes.c_int]
    lib.orc_result_dtype.argtypes = [ctypes.c_void_p, ctypes.c_int]
    lib.orc_result_rank.argtypes = [ctypes.c_void_p, ctypes.c_int]
    lib.orc_result_dims.restype = ctypes.POINTER(ctypes.c_int64)
    lib.orc_result_dims.argtypes = [ctypes.c_void_p, ctypes.c_int]
    lib.orc_result_data.restype = ctypes.c_void_p
    lib.orc_result_data.argtypes = [ctypes.c_void_p, ctypes.c_int]
    lib.orc_erfinv.restype = ctypes.c_double
    lib.orc_erfinv.argtypes = [ctypes.c_double]
    lib.orc_philox4x32_10.argtypes = [ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32),
                                     ctypes.POINTER(ctypes.c_uint32)]
    _lib = lib
    return lib


class OracleError(ValueError):
    """The interpreter raised (missing input, bad index, division by zero...)."""


class _Compiled:
    def __init__(self, graph, handle):
        self.graph = graph
        self.handle = handle

    def __del__(self):
        if self.handle and _lib is not None:
            _lib.orc_free(self.handle)
            self.handle = None


class Interp:
    """``Backend.S`` over the C oracle: ``compile`` parses the wire text,
    ``run`` evaluates it the interpreter's way."""

    name = "interp"

    @staticmethod
    def compile(g):
        lib = _load()
        err = ctypes.create_string_buffer(1024)
        h = lib.orc_parse(g.to_wire().encode(), err, 1024)
        if not h:
            raise OracleError(err.value.decode())
        return _Compiled(g, h)

    @staticmethod
    def run(c, inputs):
        lib = _load()
        items = list(inputs.items()) if isinstance(inputs, dict) else list(inputs)
        arrays = []
        names = []
        dts = []
        ranks = []
        dims = []
        datas = []
        for name, v in items:
            a = np.asarray(v, order="C")
            d = ir.dtype_of_numpy(a)
            if d is None:
                raise ValueError("Interp.run: input %r has unsupported numpy dtype %s" % (name, a.dtype))
            arrays.append(a)
            names.append(name.encode())
            dts.append(d.code)
            ranks.append(a.ndim)
            dims.append((ctypes.c_int64 * max(1, a.ndim))(*a.shape))
            datas.append(a.ctypes.data)
        n = len(items)
        err = ctypes.create_string_buffer(1024)
        res = lib.orc_run(
            c.handle, n, (ctypes.c_char_p * max(1, n))(*names), (ctypes.c_int * max(1, n))(*dts),
            (ctypes.c_int * max(1, n))(*ranks),
            (ctypes.POINTER(ctypes.c_int64) * max(1, n))(*[ctypes.cast(x, ctypes.POINTER(ctypes.c_int64)) for x in dims]),
            (ctypes.c_void_p * max(1, n))(*datas), err, 1024,
        )
        if not res:
            raise OracleError(err.value.decode())
        try:
            out = []
            for i in range(lib.orc_result_count(res)):
                name = lib.orc_result_name(res, i).decode()
                d = ir.dtype_of_code(lib.orc_result_dtype(res, i))
                rank = lib.orc_result_rank(res, i)
                dp = lib.orc_result_dims(res, i)
                shape = tuple(dp[k] for k in range(rank))
                count = ir.numel(shape)
                arr = np.empty(shape, dtype=d.np)
                if count:
                    ctypes.memmove(arr.ctypes.data, lib.orc_result_data(res, i), count * d.size)
                out.append((name, arr))
            return out
        finally:
            lib.orc_result_free(res)


def run(g, inputs):
    return Interp.run(Interp.compile(g), inputs)


def erfinv(x):
    return _load().orc_erfinv(float(x))


def philox4x32_10(ctr, key):
    lib = _load()
    c = (ctypes.c_uint32 * 4)(*[v & 0xFFFFFFFF for v in ctr])
    k = (ctypes.c_uint32 * 2)(*[v & 0xFFFFFFFF for v in key])
    o = (ctypes.c_uint32 * 4)()
    lib.orc_philox4x32_10(c, k, o)
    return [o[i] for i in range(4)]
