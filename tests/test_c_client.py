"""The C-ABI driven from plain C (tests/c_client/c_client.c): the headers
compile as strict C99, and a C client compiles, plans and runs graphs
through libcchip.so alone, as any foreign-function binding would
(Backend.S, lib/backend/backend.ml:13-20). The client is built in-tree by
``__graft_entry__.build()`` and called here through ctypes."""

import ctypes
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle
from cudacaml_amd import differential as Diff
from cudacaml_amd.examples import configs as C
from cudacaml_amd.ir import F32

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DIR = os.path.join(ROOT, "tests", "c_client")
LIB = os.path.join(DIR, "libc_client.so")
STRICT = ["-std=c99", "-pedantic", "-Wall", "-Wextra", "-Werror"]


def client():
    """The in-tree client library (built by __graft_entry__.build(); made
    here only if absent)."""
    if not os.path.exists(LIB):
        subprocess.run(["make", "-s", "-C", DIR], check=True)
    lib = ctypes.CDLL(LIB)
    lib.cclient_param_names.restype = ctypes.c_int
    lib.cclient_param_names.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]
    lib.cclient_run.restype = ctypes.c_int
    lib.cclient_run.argtypes = [
        ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_void_p),
        ctypes.POINTER(ctypes.c_size_t), ctypes.c_int, ctypes.POINTER(ctypes.c_void_p),
        ctypes.POINTER(ctypes.c_size_t), ctypes.c_char_p, ctypes.c_size_t,
    ]
    return lib


def run_c(g, inputs, outputs):
    """Runs graph `g` through the C client on `inputs` [(name, array)],
    into fresh arrays shaped like `outputs` [(name, dtype, shape)]:
    (status, message, {name: array})."""
    lib = client()
    arrs = [np.ascontiguousarray(a) for _, a in inputs]
    names = (ctypes.c_char_p * len(inputs))(*[n.encode() for n, _ in inputs])
    host = (ctypes.c_void_p * len(inputs))(*[a.ctypes.data for a in arrs])
    nbytes = (ctypes.c_size_t * len(inputs))(*[a.nbytes for a in arrs])
    outs = [np.zeros(shape, dtype=dt) for _, dt, shape in outputs]
    optr = (ctypes.c_void_p * len(outs))(*[o.ctypes.data for o in outs])
    obytes = (ctypes.c_size_t * len(outs))(*[o.nbytes for o in outs])
    msg = ctypes.create_string_buffer(1024)
    rc = lib.cclient_run(g.to_wire().encode(), len(inputs), names, host, nbytes, len(outs), optr, obytes, msg,
                         len(msg))
    return rc, msg.value.decode(), {name: o for (name, _, _), o in zip(outputs, outs)}


def test_headers_and_client_are_strict_c99(tmp_path):
    """Both headers and the client compile as C99 with -pedantic -Werror,
    with no C++ in them."""
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    tu = tmp_path / "headers.c"
    tu.write_text('#include "cchip_runtime.h"\n#include "cchip_backend.h"\nint main(void) { return 0; }\n')
    inc = "-I" + os.path.join(ROOT, "include")
    for src in (str(tu), os.path.join(DIR, "c_client.c")):
        subprocess.run([cc] + STRICT + [inc, "-fsyntax-only", src], check=True)


def test_c_client_reads_the_plan_without_a_device():
    """cchip_backend_plan from C: the params of a graph, in Graph.params
    order."""
    buf = ctypes.create_string_buffer(4096)
    assert client().cclient_param_names(C.saxpy(1 << 10).to_wire().encode(), buf, len(buf)) == 2
    assert buf.value.decode().split() == ["x", "y"]
    n = client().cclient_param_names(C.scatter_gather(1 << 10, 64).to_wire().encode(), buf, len(buf))
    assert n == 2 and sorted(buf.value.decode().split()) == ["idx", "src"]


@pytest.mark.gpu
def test_c_client_runs_saxpy_against_the_oracle(device):
    """Config 1's graph compiled and run from C: r bit for bit and s within
    the band, against the oracle."""
    n = (1 << 20) + 3
    g = C.saxpy(n)
    ins = [("x", C.uniform_pm1(1, (n,))), ("y", C.uniform_pm1(2, (n,)))]
    rc, msg, got = run_c(g, ins, [("r", np.float32, (n,)), ("s", np.float32, ())])
    assert rc == 0, msg
    exp = dict(oracle.run(g, ins))
    np.testing.assert_array_equal(got["r"], exp["r"])
    bad = [v for v in Diff.policy_check(g, list(exp.items()), list(got.items())) if not v.ok]
    assert not bad, bad


@pytest.mark.gpu
def test_c_client_runs_a_scatter_and_reports_errors(device):
    """A scatter_add with gather back from C against the oracle; then the
    errors a C caller sees: an input of the wrong size (before any device
    work) and an out-of-range index (after the run), with the interpreter's
    messages."""
    n, bins = 100003, 4099
    g = C.scatter_gather(n, bins, F32)
    idx = (C.philox_w0(21, n).astype(np.int64) % bins).astype(np.int32)
    ins = [("idx", idx), ("src", C.uniform_pm1(22, (n,)))]
    outs = [("h", np.float32, (bins,)), ("back", np.float32, (n,))]
    rc, msg, got = run_c(g, ins, outs)
    assert rc == 0, msg
    exp = dict(oracle.run(g, ins))
    bad = [v for v in Diff.policy_check(g, list(exp.items()), list(got.items())) if not v.ok]
    assert not bad, bad
    rc, msg, _ = run_c(g, [("idx", idx[:-1]), ins[1]], outs)
    assert rc != 0 and "idx" in msg, (rc, msg)
    wrong = idx.copy()
    wrong[7] = bins
    rc, msg, _ = run_c(g, [("idx", wrong), ins[1]], outs)
    assert rc != 0 and "out of bounds" in msg, (rc, msg)
