"""``Backend_hip``: the gfx950 backend behind the reference's plugin signature.

Mirrors ``Backend.S`` (``lib/backend/backend.ml:13-20``: ``name``,
``compile``, ``run``) and the extensions of ``Backend_cuda``
(``lib/backend_cuda/cudacaml_backend_cuda.mli:7-84``: ``source``,
``release``, ``executor``, ``compile_with``, ``compile_on``,
``run_async``/``wait``, residents and ``run_resident``) with the same
argument meaning and errors: a caller mistake raises ``ValueError`` (the
reference's ``Invalid_argument``), a driver/JIT/plan error ``RuntimeError``
(``Failure``). Everything below is a thin layer over the C-ABI of
``include/cchip_backend.h``; the fusion plan, the kernels and the executor
are native.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import ir
from ._lib import check, lib, take_string
from .runtime import Buffer, Device

name = "hip"


def _items(inputs):
    return list(inputs.items()) if isinstance(inputs, dict) else list(inputs)


def source(g):
    """The generated HIP source of a graph, without compiling it."""
    out = ctypes.c_void_p()
    check(lib().cchip_backend_source(g.to_wire().encode(), ctypes.byref(out)))
    return take_string(out.value)


def plan(g):
    """Buffers, kernels (with template and launch geometry) and host plan,
    one per line; needs no device."""
    out = ctypes.c_void_p()
    check(lib().cchip_backend_plan(g.to_wire().encode(), ctypes.byref(out)))
    return take_string(out.value)


class _IO:
    __slots__ = ("name", "dtype", "shape", "nbytes")

    def __init__(self, name, dtype, shape):
        self.name = name
        self.dtype = dtype
        self.shape = shape
        self.nbytes = ir.numel(shape) * dtype.size


def _io(prog, i, fn):
    nm = ctypes.c_char_p()
    dt = ctypes.c_int()
    rk = ctypes.c_int()
    dims = (ctypes.c_int64 * 8)()
    check(fn(prog, i, ctypes.byref(nm), ctypes.byref(dt), ctypes.byref(rk), dims))
    return _IO(nm.value.decode(), ir.dtype_of_code(dt.value), tuple(dims[k] for k in range(rk.value)))


class Compiled:
    """A compiled program: the JIT'd module plus one executor (stream and
    buffer pool) per lane."""

    def __init__(self, g, handle):
        self.graph_name = g.name
        self.handle = handle
        L = lib()
        self.params = [_io(handle, i, L.cchip_program_param) for i in range(L.cchip_program_num_params(handle))]
        self.outputs = [_io(handle, i, L.cchip_program_output) for i in range(L.cchip_program_num_outputs(handle))]
        self.device = L.cchip_program_device(handle)
        self.streams = L.cchip_program_streams(handle)
        self.released = False

    def kernel_names(self):
        L = lib()
        return [L.cchip_program_kernel_name(self.handle, i).decode() for i in range(L.cchip_program_kernel_count(self.handle))]

    def release(self):
        if not self.released:
            self.released = True
            check(lib().cchip_program_release(self.handle))

    def __del__(self):
        try:
            if self.handle:
                lib().cchip_program_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


class Executor:
    """The executor behind lane 0 of a compiled program (tests and tooling)."""

    def __init__(self, c):
        self._c = c

    def buffer_count(self):
        return lib().cchip_program_buffer_count(self._c.handle)

    def stream_ptr(self):
        s = ctypes.c_void_p()
        check(lib().cchip_program_stream(self._c.handle, 0, ctypes.byref(s)))
        return s.value


def compile_on(device, g, streams=1):
    if streams < 1:
        raise ValueError("Backend_hip.compile_on: streams must be >= 1")
    h = ctypes.c_void_p()
    check(lib().cchip_backend_compile(g.to_wire().encode(), device, streams, ctypes.byref(h)))
    return Compiled(g, h.value)


def compile_with(streams, g):
    return compile_on(0, g, streams=streams)


def compile(g):  # noqa: A001 - Backend.S name
    return compile_on(0, g)


def device_of(c):
    return c.device


def release(c):
    c.release()


def executor(c):
    return Executor(c)


def _bind(c, inputs, who):
    """Check names, dtypes and shapes the way the interpreter does, and return
    the arrays in a ctypes-ready form (all host memory stays referenced)."""
    items = _items(inputs)
    by_name = {}
    for n, v in items:
        by_name.setdefault(n, v)
    names, ptrs, sizes, keep = [], [], [], []
    for p in c.params:
        if p.name not in by_name:
            raise ValueError("%s: missing input %s" % (who, p.name))
        v = by_name[p.name]
        a = np.asarray(v, order="C")
        d = ir.dtype_of_numpy(a)
        if d is not p.dtype:
            raise ValueError("%s: input %r has dtype %s, expected %s" % (who, p.name, d.name if d else a.dtype, p.dtype.name))
        if tuple(a.shape) != p.shape:
            raise ValueError("%s: input %r has shape %s, expected %s" % (
                who, p.name, ir.shape_to_string(a.shape), ir.shape_to_string(p.shape)))
        keep.append(a)
        names.append(p.name.encode())
        ptrs.append(a.ctypes.data)
        sizes.append(a.nbytes)
    n = len(names)
    return (n, (ctypes.c_char_p * max(1, n))(*names), (ctypes.c_void_p * max(1, n))(*ptrs),
            (ctypes.c_size_t * max(1, n))(*sizes), keep)


def _fresh_outputs(c):
    outs = [np.empty(o.shape, dtype=o.dtype.np) for o in c.outputs]
    arr = (ctypes.c_void_p * max(1, len(outs)))(*[o.ctypes.data for o in outs])
    return outs, arr


def run(c, inputs):
    """Synchronous run on lane 0; outputs are fresh arrays in Graph.outputs
    order, keyed by name."""
    if c.released:
        raise RuntimeError("Executor.run: this executor has been released")
    n, names, ptrs, sizes, keep = _bind(c, inputs, "Executor.run")
    outs, arr = _fresh_outputs(c)
    check(lib().cchip_program_run(c.handle, n, names, ptrs, sizes, arr))
    del keep
    return [(o.name, v) for o, v in zip(c.outputs, outs)]


class Job:
    __slots__ = ("c", "handle", "outs", "keep", "result")

    def __del__(self):
        try:
            if self.handle:
                lib().cchip_job_free(self.handle)
        except Exception:
            pass


def run_async(c, inputs):
    """Issue a run on the next lane and return; the job owns its input and
    output host memory until it has been waited on."""
    if c.released:
        raise RuntimeError("Executor.run: this executor has been released")
    n, names, ptrs, sizes, keep = _bind(c, inputs, "Executor.run")
    outs, arr = _fresh_outputs(c)
    h = ctypes.c_void_p()
    check(lib().cchip_program_run_async(c.handle, n, names, ptrs, sizes, arr, ctypes.byref(h)))
    j = Job()
    j.c = c
    j.handle = h.value
    j.outs = outs
    j.keep = (keep, names, ptrs, sizes, arr)
    j.result = None
    return j


def wait(j):
    """Block until the job's downloads are done; waiting twice is harmless."""
    if j.result is None:
        check(lib().cchip_job_wait(j.handle))
        j.result = [(o.name, v) for o, v in zip(j.c.outputs, j.outs)]
        j.keep = None
    return j.result


# ---------------------------------------------------------------------------
# Device-resident values
# ---------------------------------------------------------------------------


class Resident:
    """A device buffer plus the dtype and shape that interpret it."""

    __slots__ = ("buf", "dtype", "shape")

    def __init__(self, buf, dtype, shape):
        self.buf = buf
        self.dtype = dtype
        self.shape = tuple(shape)


def upload(v):
    a = np.asarray(v, order="C")
    d = ir.dtype_of_numpy(a)
    if d is None:
        raise ValueError("Backend_hip.upload: unsupported dtype %s" % a.dtype)
    b = Buffer.alloc(a.nbytes)
    b.upload(a)
    return Resident(b, d, a.shape)


def download(r):
    v = np.empty(r.shape, dtype=r.dtype.np)
    r.buf.download(v)
    return v


def free_resident(r):
    r.buf.free()


def _bind_resident(c, inputs, who):
    by_name = {}
    for n, r in _items(inputs):
        by_name.setdefault(n, r)
    names, ptrs, sizes = [], [], []
    for p in c.params:
        if p.name not in by_name:
            raise ValueError("%s: missing input %s" % (who, p.name))
        r = by_name[p.name]
        names.append(p.name.encode())
        ptrs.append(r.buf.ptr)
        sizes.append(r.buf.nbytes)
    n = len(names)
    return (n, (ctypes.c_char_p * max(1, n))(*names), (ctypes.c_void_p * max(1, n))(*ptrs),
            (ctypes.c_size_t * max(1, n))(*sizes))


def run_resident(c, inputs):
    """Device in, device out: inputs are residents bound by name (exact byte
    size), outputs are fresh residents the caller owns. Synchronises."""
    if c.released:
        raise RuntimeError("Executor.run_resident: this executor has been released")
    n, names, ptrs, sizes = _bind_resident(c, inputs, "Executor.run_resident")
    outs = (ctypes.c_void_p * max(1, len(c.outputs)))()
    check(lib().cchip_program_run_resident(c.handle, n, names, ptrs, sizes, outs))
    return [(o.name, Resident(Buffer(outs[i], o.nbytes), o.dtype, o.shape)) for i, o in enumerate(c.outputs)]


def _bind_outputs(c, outputs):
    by_name = dict(_items(outputs))
    ptr_out = []
    for o in c.outputs:
        r = by_name.get(o.name)
        if r is None:
            raise ValueError("Executor.run_resident: missing output buffer %s" % o.name)
        if r.buf.nbytes != o.nbytes:
            raise ValueError("Executor.run_resident: output %s is %d bytes, needs %d" % (o.name, r.buf.nbytes, o.nbytes))
        ptr_out.append(r.buf.ptr)
    return (ctypes.c_void_p * max(1, len(ptr_out)))(*ptr_out)


def run_resident_into(c, inputs, outputs, sync=True):
    """Extension (no reference counterpart): like ``run_resident`` but into
    caller-owned output residents, optionally without synchronising."""
    if c.released:
        raise RuntimeError("Executor.run_resident: this executor has been released")
    n, names, ptrs, sizes = _bind_resident(c, inputs, "Executor.run_resident")
    arr = _bind_outputs(c, outputs)
    check(lib().cchip_program_run_resident_into(c.handle, n, names, ptrs, sizes, arr, 1 if sync else 0))


def run_resident_noalloc(c, inputs, outputs, stream=None, err=None):
    """Extension (no reference counterpart), for callers that cannot
    allocate device memory: ``run_resident_into`` without synchronising, on
    ``stream`` (a raw HIP stream pointer; None is the default stream), with
    the template scratch taken from the library's static 32 MiB array.
    Only issues the work: synchronise the stream before reading outputs.
    ``err``, a device buffer of at least 4 bytes the caller owns, receives
    this call's device-side error word (0: none; ``raise_error_word``
    turns it into the exception a synchronous run raises); without it the
    call's index errors are dropped, never reported by another run."""
    if c.released:
        raise RuntimeError("Executor.run_resident: this executor has been released")
    n, names, ptrs, sizes = _bind_resident(c, inputs, "Executor.run_resident")
    arr = _bind_outputs(c, outputs)
    if err is not None and err.nbytes < 4:
        raise ValueError("run_resident_noalloc: the error buffer needs 4 bytes")
    check(lib().cchip_program_run_resident_noalloc(c.handle, n, names, ptrs, sizes, arr, stream,
                                                   None if err is None else err.ptr))


def raise_error_word(code):
    """Raise what a synchronous run raises for the device error flags
    ``code`` (an allocation-free call's error word); nothing for 0."""
    check(lib().cchip_error_word_status(int(code)))


def time_kernel(c, kernel_name):
    """Record timing events around every lane-0 launch of ``kernel_name``."""
    check(lib().cchip_program_time_kernel(c.handle, kernel_name.encode() if kernel_name else None))


def timing(c):
    """(launches, summed milliseconds) of the timed kernel since the last read."""
    n = ctypes.c_int()
    ms = ctypes.c_double()
    check(lib().cchip_program_timing(c.handle, ctypes.byref(n), ctypes.byref(ms)))
    return n.value, ms.value


def timing_each(c, capacity=4096):
    """Per-launch milliseconds of the timed kernel since the last read, in
    launch order."""
    buf = (ctypes.c_double * capacity)()
    n = ctypes.c_int()
    ms = ctypes.c_double()
    check(lib().cchip_program_timing_each(c.handle, capacity, buf, ctypes.byref(n), ctypes.byref(ms)))
    return list(buf[:min(n.value, capacity)])


available = Device.available
