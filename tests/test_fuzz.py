"""Seeded random graphs (tests/fuzz_graphs.py), no GPU needed: each graph
runs on the oracle and its generated HIP module compiles for gfx950."""

import pytest

import oracle
from cudacaml_amd import backend_hip as H
from cudacaml_amd import runtime

import fuzz_graphs as FG

N_CASES = 100


@pytest.mark.parametrize("seed", range(N_CASES))
def test_fuzz_graph_builds_runs_and_compiles(seed):
    name, g, inputs = FG.case(seed)
    outs = oracle.run(g, inputs)
    assert [n for n, _ in outs] == [n for n, _ in g.outputs]
    assert runtime.Jit.check(name, H.source(g)) > 0
