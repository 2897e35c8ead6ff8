"""The C-ABI library loads and exports every function that include/*.h
declares, and the Python bindings declare exactly those. No GPU: nothing
here launches or allocates."""

import ctypes
import os
import re

from cudacaml_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    names = set()
    for h in ("cchip_runtime.h", "cchip_backend.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(cchip_[a-z_0-9]+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_every_declared_symbol_is_exported():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in sorted(declared()) if not hasattr(lib, n)]
    assert not missing, missing


def test_bindings_cover_the_headers():
    assert declared() == set(_lib.SIGNATURES)


def test_no_device_queries_are_safe():
    from cudacaml_amd.runtime import Device

    assert Device.available() in (True, False)
    assert _lib.lib().cchip_buffer_live_count() >= 0


def test_error_word_status_gives_the_interpreters_messages():
    """The allocation-free call's error word maps to the exceptions a
    synchronous run raises; no device is touched."""
    import pytest

    from cudacaml_amd import backend_hip as H

    H.raise_error_word(0)
    with pytest.raises(ValueError, match="gather index out of bounds"):
        H.raise_error_word(1)
    with pytest.raises(ValueError, match="scatter_add index out of bounds"):
        H.raise_error_word(2)
    with pytest.raises(ValueError, match="look-back did not complete"):
        H.raise_error_word(4)
