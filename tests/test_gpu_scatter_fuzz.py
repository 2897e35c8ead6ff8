"""Seeded random scatter_add + gather-back graphs on the device against the
oracle: sizes, bin counts, dtypes and index distributions drawn so that
every scatter layout is taken (one slice folded directly, tile-local runs,
counted chunks, two levels with the slice pass in windows, the gather's
slice step inside the accumulate or as its own kernel), each also under
the knob that switches the layout off. The per-output policy applies
(integers bit-exact, float sums within the accumulation band), and the
gather back must be exactly h[idx]."""

import numpy as np
import pytest

import oracle
from cudacaml_amd import backend_hip as H
from cudacaml_amd import differential as Diff
from cudacaml_amd.examples import configs as C
from cudacaml_amd.ir import F32, F64, I32

pytestmark = pytest.mark.gpu

N_CASES = 24
KNOBS = ["", "scatter_windows=0", "scatter_fuse_back=0", "scatter_local_max=0"]


def case(seed):
    r = np.random.default_rng(1000 + seed)
    dt = [F32, I32, F64][seed % 3]
    n = int(2 ** r.uniform(10, 22)) + int(r.integers(0, 9))
    bins = int(2 ** r.uniform(12, 25)) + int(r.integers(0, 5))
    kind = ["uniform", "crowded", "bands", "permutation"][(seed // 3) % 4]
    if kind == "permutation" and bins >= n:
        idx = r.permutation(bins)[:n]
    elif kind == "crowded":
        idx = np.where(r.random(n) < 0.3, bins // 3, r.integers(0, bins, n))
    elif kind == "bands":
        lo = r.integers(0, max(1, bins - 4096))
        idx = np.where(r.random(n) < 0.7, r.integers(lo, min(bins, lo + 4096), n),
                       r.integers(max(0, bins - 100), bins, n))
    else:
        idx = r.integers(0, bins, n)
    idx = idx.astype(np.int32)
    if dt is I32:
        src = r.integers(-50, 50, n).astype(np.int32)
    else:
        src = r.uniform(0.0, 1.0, n).astype(dt.np)  # positive: sums stay clear of zero
    return dt, n, bins, kind, [("idx", idx), ("src", src)]


@pytest.mark.parametrize("seed", range(N_CASES))
def test_scatter_gather_fuzz(device, monkeypatch, seed):
    dt, n, bins, kind, inputs = case(seed)
    monkeypatch.setenv("CCHIP_TUNE", KNOBS[seed % len(KNOBS)])
    g = C.scatter_gather(n, bins, dt)
    print("case", seed, dt.name, n, bins, kind, KNOBS[seed % len(KNOBS)], flush=True)
    exp = oracle.run(g, inputs)
    c = H.compile(g)
    try:
        got = H.run(c, inputs)
    finally:
        c.release()
    bad = [v for v in Diff.policy_check(g, exp, got) if not v.ok]
    assert not bad, (seed, bad)
    o = dict(got)
    np.testing.assert_array_equal(o["back"], o["h"][inputs[0][1]])
