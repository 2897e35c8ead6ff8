"""The runtime seen from Python: ``Device``, ``Buffer``, ``Stream``,
``Event``, ``Jit``, ``Launch`` and ``Pinned``, mirroring the OCaml modules of
``lib/runtime`` (``device.mli``, ``buffer.mli``, ``stream.mli``,
``event.mli``, ``jit.mli``, ``launch.mli``, ``pinned.mli``) over the C-ABI
of ``include/cchip_runtime.h``.

Host values are numpy arrays (the reference's Bigarray-backed ``Value.t``).
"""

from __future__ import annotations

import contextlib
import ctypes
import weakref

import numpy as np

from . import ir
from ._lib import check, lib

# ---------------------------------------------------------------------------
# Device
# ---------------------------------------------------------------------------


class Device:
    @staticmethod
    def available():
        """False on machines with no usable HIP device; never raises."""
        try:
            return bool(lib().cchip_device_available())
        except Exception:
            return False

    @staticmethod
    def init():
        check(lib().cchip_device_init())

    @staticmethod
    def synchronize():
        check(lib().cchip_device_synchronize())

    @staticmethod
    def count():
        n = ctypes.c_int()
        check(lib().cchip_device_count(ctypes.byref(n)))
        return n.value

    @staticmethod
    def current():
        d = ctypes.c_int()
        check(lib().cchip_device_get(ctypes.byref(d)))
        return d.value

    @staticmethod
    @contextlib.contextmanager
    def with_device(ordinal):
        """Make ``ordinal`` current for the block; restores the previous one
        even on exceptions (device.ml:59-79)."""
        prev = Device.current()
        check(lib().cchip_device_set(ordinal))
        try:
            yield
        finally:
            lib().cchip_device_set(prev)

    class Info:
        __slots__ = ("name", "arch", "multiprocessors", "total_memory_bytes")

        def __init__(self, name, arch, mps, mem):
            self.name = name
            self.arch = arch
            self.multiprocessors = mps
            self.total_memory_bytes = mem

    @staticmethod
    def info_of(ordinal):
        name = ctypes.create_string_buffer(256)
        arch = ctypes.create_string_buffer(64)
        mps = ctypes.c_int()
        mem = ctypes.c_int64()
        check(lib().cchip_device_info(ordinal, name, 256, arch, 64, ctypes.byref(mps), ctypes.byref(mem)))
        return Device.Info(name.value.decode(), arch.value.decode(), mps.value, mem.value)

    @staticmethod
    def info():
        return Device.info_of(0)

    @staticmethod
    def name():
        return Device.info().name

    @staticmethod
    def info_to_string(i):
        """Four grep-able lines (device.mli:47-56); the compute line names the
        gfx architecture where CUDA printed sm_XY."""
        return "device: %s\ncompute: %s\nmultiprocessors: %d\nmemory_mib: %d\n" % (
            i.name, i.arch, i.multiprocessors, i.total_memory_bytes // 1048576)


# ---------------------------------------------------------------------------
# Stream and Event
# ---------------------------------------------------------------------------


class Stream:
    """A HIP stream. ``Stream.default`` is the NULL stream; ``create`` makes a
    non-blocking one at the default priority."""

    __slots__ = ("ptr", "_owned", "__weakref__")

    def __init__(self, ptr, owned):
        self.ptr = ptr
        self._owned = owned

    @staticmethod
    def create():
        s = ctypes.c_void_p()
        check(lib().cchip_stream_create(ctypes.byref(s)))
        st = Stream(s.value, True)
        weakref.finalize(st, _destroy_stream, s.value)
        return st

    def synchronize(self):
        check(lib().cchip_stream_synchronize(self.ptr))

    def is_idle(self):
        i = ctypes.c_int()
        check(lib().cchip_stream_is_idle(self.ptr, ctypes.byref(i)))
        return bool(i.value)


def _destroy_stream(p):
    try:
        lib().cchip_stream_destroy(p)
    except Exception:
        pass


Stream.default = Stream(None, False)


class Event:
    __slots__ = ("ptr", "__weakref__")

    def __init__(self, ptr):
        self.ptr = ptr
        weakref.finalize(self, _destroy_event, ptr)

    @staticmethod
    def record(stream=None):
        stream = stream or Stream.default
        e = ctypes.c_void_p()
        check(lib().cchip_event_record(stream.ptr, ctypes.byref(e)))
        return Event(e.value)

    def wait(self, stream):
        check(lib().cchip_event_wait(stream.ptr, self.ptr))

    def synchronize(self):
        check(lib().cchip_event_synchronize(self.ptr))

    @staticmethod
    def elapsed_ms(start, stop):
        ms = ctypes.c_float()
        check(lib().cchip_event_elapsed_ms(start.ptr, stop.ptr, ctypes.byref(ms)))
        return ms.value


def _destroy_event(p):
    try:
        lib().cchip_event_destroy(p)
    except Exception:
        pass


# ---------------------------------------------------------------------------
# Buffer
# ---------------------------------------------------------------------------


def _host_ptr(v):
    if not isinstance(v, np.ndarray) or not v.flags["C_CONTIGUOUS"]:
        raise ValueError("Buffer: host values must be C-contiguous numpy arrays")
    return v.ctypes.data


class Buffer:
    """An opaque device pointer plus a byte count (buffer.mli)."""

    __slots__ = ("ptr", "nbytes", "_freed")

    def __init__(self, ptr, nbytes):
        self.ptr = ptr
        self.nbytes = nbytes
        self._freed = False

    @staticmethod
    def alloc(nbytes):
        p = ctypes.c_void_p()
        check(lib().cchip_buffer_alloc(nbytes, ctypes.byref(p)))
        return Buffer(p.value, nbytes)

    def free(self):
        if not self._freed:
            self._freed = True
            check(lib().cchip_buffer_free(self.ptr))

    def byte_size(self):
        return self.nbytes

    @staticmethod
    def live_count():
        return lib().cchip_buffer_live_count()

    def _same(self, v):
        if v.nbytes != self.nbytes:
            raise ValueError("Buffer: host value has %d bytes, buffer has %d" % (v.nbytes, self.nbytes))

    def upload(self, v):
        self._same(v)
        check(lib().cchip_buffer_upload(self.ptr, _host_ptr(v), v.nbytes))

    def download(self, v):
        self._same(v)
        check(lib().cchip_buffer_download(_host_ptr(v), self.ptr, v.nbytes))

    def upload_async(self, v, stream):
        self._same(v)
        check(lib().cchip_buffer_upload_async(self.ptr, _host_ptr(v), v.nbytes, stream.ptr))

    def download_async(self, v, stream):
        self._same(v)
        check(lib().cchip_buffer_download_async(_host_ptr(v), self.ptr, v.nbytes, stream.ptr))

    @staticmethod
    def copy_device(dst, src, stream=None):
        if dst.nbytes != src.nbytes:
            raise ValueError("Buffer.copy_device: sizes differ (%d vs %d)" % (dst.nbytes, src.nbytes))
        check(lib().cchip_buffer_copy_device(dst.ptr, src.ptr, src.nbytes, (stream or Stream.default).ptr))


# ---------------------------------------------------------------------------
# Jit and Launch
# ---------------------------------------------------------------------------


class Module:
    __slots__ = ("ptr", "name")

    def __init__(self, ptr, name):
        self.ptr = ptr
        self.name = name


class Jit:
    @staticmethod
    def compile(name, source):
        m = ctypes.c_void_p()
        check(lib().cchip_jit_compile(name.encode(), source.encode(), ctypes.byref(m)))
        return Module(m.value, name)

    @staticmethod
    def check(name, source):
        """Compile only (no device): the code object's size in bytes."""
        n = ctypes.c_size_t()
        check(lib().cchip_jit_check(name.encode(), source.encode(), ctypes.byref(n)))
        return n.value

    @staticmethod
    def code_size(m):
        n = ctypes.c_size_t()
        check(lib().cchip_jit_code_size(m.ptr, ctypes.byref(n)))
        return n.value

    @staticmethod
    def get_kernel(m, name):
        k = ctypes.c_void_p()
        check(lib().cchip_jit_get_kernel(m.ptr, name.encode(), ctypes.byref(k)))
        return k.value

    @staticmethod
    def unload(m):
        check(lib().cchip_jit_unload(m.ptr))


class Launch:
    @staticmethod
    def run(kernel, grid, block, bufs, grid_y=1, block_y=1, shared_bytes=0, stream=None):
        n = len(bufs)
        arr = (ctypes.c_void_p * max(1, n))(*[b.ptr for b in bufs])
        check(lib().cchip_launch(kernel, grid, grid_y, block, block_y, shared_bytes,
                                 (stream or Stream.default).ptr, n, arr))


# ---------------------------------------------------------------------------
# Pinned
# ---------------------------------------------------------------------------


def _free_pinned(p):
    try:
        lib().cchip_pinned_free(p)
    except Exception:
        pass


class Pinned:
    """Page-locked host memory as numpy arrays (pinned.mli:17-33). The
    array's base owns the allocation and frees it when the last view dies."""

    @staticmethod
    def alloc(dtype, shape):
        if dtype is ir.BOOL:
            raise ValueError("Pinned.alloc: Bool tensors are not storable")
        count = ir.numel(shape)
        n = count * dtype.size
        p = ctypes.c_void_p()
        check(lib().cchip_pinned_alloc(n, ctypes.byref(p)))

        class _Owned(ctypes.c_char * max(1, n)):
            def __del__(self):
                _free_pinned(self._cchip_ptr)

        raw = _Owned.from_address(p.value)
        raw._cchip_ptr = p.value
        return np.frombuffer(raw, dtype=dtype.np, count=count).reshape(shape)

    @staticmethod
    def of_value(v):
        d = ir.dtype_of_numpy(v)
        if d is None:
            raise ValueError("Pinned.of_value: unsupported dtype %s" % v.dtype)
        a = Pinned.alloc(d, v.shape)
        a[...] = v
        return a

    @staticmethod
    def is_pinned(v):
        if not isinstance(v, np.ndarray):
            return False
        return bool(lib().cchip_pinned_is_pinned(ctypes.c_void_p(v.ctypes.data)))
