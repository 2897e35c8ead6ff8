"""The f32 element-wise functions against the oracle, densely.

The interpreter computes every f32 unary op in double and rounds once (R1,
lib/backend_interp/cudacaml_backend_interp.ml:145-160). The device does
the same: exp and log with its own double-precision evaluations (cc_expf,
cc_logf), sin, cos and erf through the device library's double-precision
functions, sqrt with the correctly rounded f32 instruction; erfinv is its
own single-precision fit (within 2 ulp, tested in test_gpu_parity.py).
Each function is swept over every 251st float of the whole finite range,
both signs, plus the special values, and over 2^24 random bit patterns:
the same bits as the oracle everywhere (NaN where the oracle gives NaN),
well inside the 2-ulp bar."""

import numpy as np
import pytest

import oracle
from cudacaml_amd import backend_hip as H
from cudacaml_amd import differential as Diff
from cudacaml_amd import dsl as D
from cudacaml_amd.ir import F32, Graph

pytestmark = pytest.mark.gpu

SPECIAL = np.array([0x00000000, 0x00000001, 0x007FFFFF, 0x00800000, 0x3F800000, 0x3F7FFFFF, 0x3F800001,
                    0x40490FDB, 0x3FC90FDB, 0x4B000000, 0x7F7FFFFF, 0x7F800000, 0x7FC00000], dtype=np.uint32)


def sweep_points():
    pos = np.concatenate([np.arange(0, 0x7F800001, 251, dtype=np.int64).astype(np.uint32), SPECIAL]).view(np.float32)
    return np.concatenate([pos, -pos])


@pytest.mark.parametrize("fn", ["exp", "log", "sin", "cos", "erf", "sqrt"])
def test_f32_function_dense_sweep(device, fn):
    rnd = np.random.default_rng(31).integers(0, 1 << 32, size=1 << 24, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([sweep_points(), rnd.view(np.float32)])
    g = Graph.create(fn, [("r", D.map(getattr(D, fn), D.param("x", F32, (x.size,))))])
    e = dict(oracle.run(g, [("x", x)]))["r"]
    c = H.compile(g)
    try:
        r = dict(H.run(c, [("x", x)]))["r"]
    finally:
        c.release()
    d = Diff.ulp_distance_f32(e, r)
    i = int(np.argmax(d))
    assert int(d[i]) <= 2, (fn, float(x[i]), hex(int(x[i:i + 1].view(np.uint32)[0])), float(e[i]), float(r[i]))
    np.testing.assert_array_equal(np.isnan(r), np.isnan(e))
    same = (e.view(np.uint32) == r.view(np.uint32)) | (np.isnan(e) & np.isnan(r))
    j = int(np.argmin(same))
    assert same.all(), (fn, int((~same).sum()), hex(int(x[j:j + 1].view(np.uint32)[0])), float(e[j]), float(r[j]))
