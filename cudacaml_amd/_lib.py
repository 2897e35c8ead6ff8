"""Loads ``libcchip.so`` and declares the C-ABI of ``include/cchip_*.h``.

There is no fallback: if the library is missing the import of anything that
needs it raises, so a GPU run can never silently take another path.
"""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# CCHIP_LIB selects another build of the same library (the host-sanitized
# one of build.py); by default the in-tree libcchip.so.
LIB_PATH = os.environ.get("CCHIP_LIB") or os.path.join(HERE, "libcchip.so")

OK = 0
INVALID_ARGUMENT = 1
FAILURE = 2

c_int = ctypes.c_int
c_size = ctypes.c_size_t
c_vp = ctypes.c_void_p
c_cp = ctypes.c_char_p
c_i64 = ctypes.c_int64
P = ctypes.POINTER

# name -> (restype, argtypes); every symbol the headers declare.
SIGNATURES = {
    # cchip_runtime.h
    "cchip_last_error": (c_cp, []),
    "cchip_device_available": (c_int, []),
    "cchip_device_init": (c_int, []),
    "cchip_device_synchronize": (c_int, []),
    "cchip_device_count": (c_int, [P(c_int)]),
    "cchip_device_get": (c_int, [P(c_int)]),
    "cchip_device_set": (c_int, [c_int]),
    "cchip_device_info": (c_int, [c_int, c_cp, c_size, c_cp, c_size, P(c_int), P(c_i64)]),
    "cchip_buffer_alloc": (c_int, [c_size, P(c_vp)]),
    "cchip_buffer_free": (c_int, [c_vp]),
    "cchip_buffer_live_count": (c_i64, []),
    "cchip_buffer_upload": (c_int, [c_vp, c_vp, c_size]),
    "cchip_buffer_download": (c_int, [c_vp, c_vp, c_size]),
    "cchip_buffer_upload_async": (c_int, [c_vp, c_vp, c_size, c_vp]),
    "cchip_buffer_download_async": (c_int, [c_vp, c_vp, c_size, c_vp]),
    "cchip_buffer_copy_device": (c_int, [c_vp, c_vp, c_size, c_vp]),
    "cchip_stream_create": (c_int, [P(c_vp)]),
    "cchip_stream_destroy": (c_int, [c_vp]),
    "cchip_stream_synchronize": (c_int, [c_vp]),
    "cchip_stream_is_idle": (c_int, [c_vp, P(c_int)]),
    "cchip_event_record": (c_int, [c_vp, P(c_vp)]),
    "cchip_event_wait": (c_int, [c_vp, c_vp]),
    "cchip_event_synchronize": (c_int, [c_vp]),
    "cchip_event_elapsed_ms": (c_int, [c_vp, c_vp, P(ctypes.c_float)]),
    "cchip_event_destroy": (c_int, [c_vp]),
    "cchip_jit_compile": (c_int, [c_cp, c_cp, P(c_vp)]),
    "cchip_jit_check": (c_int, [c_cp, c_cp, P(c_size)]),
    "cchip_jit_code_size": (c_int, [c_vp, P(c_size)]),
    "cchip_jit_get_kernel": (c_int, [c_vp, c_cp, P(c_vp)]),
    "cchip_jit_unload": (c_int, [c_vp]),
    "cchip_launch": (c_int, [c_vp, c_int, c_int, c_int, c_int, c_int, c_vp, c_int, P(c_vp)]),
    "cchip_pinned_alloc": (c_int, [c_size, P(c_vp)]),
    "cchip_pinned_free": (c_int, [c_vp]),
    "cchip_pinned_is_pinned": (c_int, [c_vp]),
    # cchip_backend.h
    "cchip_backend_source": (c_int, [c_cp, P(c_vp)]),
    "cchip_backend_plan": (c_int, [c_cp, P(c_vp)]),
    "cchip_free": (None, [c_vp]),
    "cchip_backend_compile": (c_int, [c_cp, c_int, c_int, P(c_vp)]),
    "cchip_program_release": (c_int, [c_vp]),
    "cchip_program_destroy": (c_int, [c_vp]),
    "cchip_program_device": (c_int, [c_vp]),
    "cchip_program_streams": (c_int, [c_vp]),
    "cchip_program_buffer_count": (c_int, [c_vp]),
    "cchip_program_kernel_count": (c_int, [c_vp]),
    "cchip_program_kernel_name": (c_cp, [c_vp, c_int]),
    "cchip_program_num_params": (c_int, [c_vp]),
    "cchip_program_param": (c_int, [c_vp, c_int, P(c_cp), P(c_int), P(c_int), P(c_i64)]),
    "cchip_program_num_outputs": (c_int, [c_vp]),
    "cchip_program_output": (c_int, [c_vp, c_int, P(c_cp), P(c_int), P(c_int), P(c_i64)]),
    "cchip_program_run": (c_int, [c_vp, c_int, P(c_cp), P(c_vp), P(c_size), P(c_vp)]),
    "cchip_program_run_async": (c_int, [c_vp, c_int, P(c_cp), P(c_vp), P(c_size), P(c_vp), P(c_vp)]),
    "cchip_job_wait": (c_int, [c_vp]),
    "cchip_job_free": (c_int, [c_vp]),
    "cchip_program_run_resident": (c_int, [c_vp, c_int, P(c_cp), P(c_vp), P(c_size), P(c_vp)]),
    "cchip_program_run_resident_into": (c_int, [c_vp, c_int, P(c_cp), P(c_vp), P(c_size), P(c_vp), c_int]),
    "cchip_program_run_resident_noalloc": (c_int, [c_vp, c_int, P(c_cp), P(c_vp), P(c_size), P(c_vp), c_vp, c_vp]),
    "cchip_error_word_status": (c_int, [c_int]),
    "cchip_program_stream": (c_int, [c_vp, c_int, P(c_vp)]),
    "cchip_program_time_kernel": (c_int, [c_vp, c_cp]),
    "cchip_program_timing": (c_int, [c_vp, P(c_int), P(ctypes.c_double)]),
    "cchip_program_timing_each": (c_int, [c_vp, c_int, P(ctypes.c_double), P(c_int), P(ctypes.c_double)]),
}

_lib = None


class NativeLibraryMissing(RuntimeError):
    pass


def lib():
    """The loaded library; raises if it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise NativeLibraryMissing(
            "cudacaml_amd: %s is not built; run __graft_entry__.build() or python -m cudacaml_amd.build" % LIB_PATH
        )
    L = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def check(rc):
    """Map a status to the reference's exceptions: Invalid_argument ->
    ValueError, Failure -> RuntimeError."""
    if rc == OK:
        return
    msg = lib().cchip_last_error().decode(errors="replace")
    if rc == INVALID_ARGUMENT:
        raise ValueError(msg)
    raise RuntimeError(msg)


def take_string(ptr):
    """Copy and free a malloc'd C string returned through an out-pointer."""
    try:
        return ctypes.string_at(ptr).decode()
    finally:
        lib().cchip_free(ptr)
