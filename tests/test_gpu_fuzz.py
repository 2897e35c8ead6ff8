"""Differential check of seeded random graphs (tests/fuzz_graphs.py) on the
device against the oracle, under the per-output policy: integers
bit-exact, f32 element-wise within 2 ulp, accumulations within 1e-4,
f64 within 1e-12."""

import pytest

import oracle
from cudacaml_amd import backend_hip as H
from cudacaml_amd import differential as Diff

import fuzz_graphs as FG
from test_fuzz import N_CASES

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(N_CASES))
def test_fuzz_graph_on_device(device, seed):
    name, g, inputs = FG.case(seed)
    exp = oracle.run(g, inputs)
    c = H.compile(g)
    try:
        got = H.run(c, inputs)
    finally:
        c.release()
    bad = [v for v in Diff.policy_check(g, exp, got) if not v.ok]
    assert not bad, (name, bad)
